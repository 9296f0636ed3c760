"""Causal algebraic attention on MI355X: drop-in for ``algebraic.kernels.flash``.

Mirrors the reference's public entry point ``flash_attention`` and its helpers
(src/algebraic/kernels/flash.py:59-73 Variant, 732-760 make_variant, 763-857
flash_attention, 708-729 the custom VJP) over torch tensors on the GPU, with the
arithmetic in hand-written gfx950 HIP kernels behind libalgebraic_hip.so:

* prologue ``q_s = round(q*alpha)``, ``sink/c`` and the range guard (flash.py:823-849)
  run as one HIP pass; the guard's branch (flash.py:853-856) is chosen on the device, so
  the call never synchronises with the host;
* forward / backward are the HIP kernels; the chain rule through ``q_s`` and the sink's
  ``1/c`` happen inside the backward kernels and here respectively.

Schedule knobs of the TPU kernels (``block*``, ``compact_stat``, ``resident_bwd``,
``diagonal_*``, ``head_resident``) do not change the maths; they are validated exactly as
the reference validates them and otherwise ignored. ``kind="softmax"`` and
``poly_rho=True`` are outside the algebraic hot path and raise NotImplementedError.
"""

import math
from typing import NamedTuple, Optional

import torch

from .. import _lib


class Variant(NamedTuple):
    """Static kernel variant (flash.py:59-73)."""
    kind: str
    n: int = 16
    shift: bool = True
    fast_rho: bool = False
    clamp: float = 0.0
    inv_stat: bool = False
    compact_stat: bool = False
    poly_rho: bool = False
    bounded_scores: bool = False
    resident_bwd: bool = False
    diagonal_bwd: bool = False
    diagonal_fwd: bool = False
    head_resident: bool = False
    precise_output: bool = False


def _root(value: float, n: int) -> float:
    """value^(1/n) for n a power of two, by repeated square roots (flash.py:117-123)."""
    out = float(value)
    while n > 1:
        out = math.sqrt(out)
        n //= 2
    return out


def make_variant(kind: str, n: int = 16, c: float = 16.0, seq_len: int = 2048,
                 shift: Optional[bool] = None, fast_rho: Optional[bool] = None,
                 inv_stat: Optional[bool] = None, compact_stat: bool = True,
                 poly_rho: bool = False) -> Variant:
    """Same validation and defaults as flash.py:732-760."""
    if kind == "softmax":
        return Variant("softmax", compact_stat=bool(compact_stat))
    if kind != "asinh":
        raise ValueError(f"unknown attention kernel: {kind}")
    if n < 2 or n & (n - 1):
        raise ValueError("asinh kernel needs n to be a power of two")
    if not math.isfinite(c) or c <= 0:
        raise ValueError("asinh scale c must be positive and finite")
    t = _root(1e37 / (seq_len + 1), n)
    clamp = 0.5 * (t - 1.0 / t)
    if shift is None:
        shift = clamp < 20.0
    if fast_rho is None:
        fast_rho = True
    if inv_stat is None:
        inv_stat = not shift
    if inv_stat and shift:
        raise ValueError("inverse-denominator statistic requires shift=False")
    if poly_rho and (shift or n != 16):
        raise ValueError("bounded radical approximation requires shift=False and n=16")
    return Variant("asinh", int(n), bool(shift), bool(fast_rho), float(clamp),
                   bool(inv_stat), bool(compact_stat), bool(poly_rho))


_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


class _Plan(NamedTuple):
    variant: int        # _lib.ATTN_*
    n: int
    c: float
    clamp: float
    fast_rho: bool
    inv_stat: bool
    range_guard: bool
    layout: int = 0     # _lib.LAYOUT_BHTD or _lib.LAYOUT_BTHD


class _FlashFn(torch.autograd.Function):
    """Custom VJP of flash.py:708-729 over the HIP kernels."""

    @staticmethod
    def forward(ctx, q, k, v, sink_logit, plan: _Plan):
        B, H, T, D = _bhtd(q.shape, plan.layout)
        lib = _lib.load()
        dt = _DTYPES[q.dtype]
        dev = q.device
        st = _lib.stream_of(q)
        q, k, v = _lib.aligned16(q), _lib.aligned16(k), _lib.aligned16(v)
        has_sink = sink_logit is not None
        sink_in = None
        if has_sink:
            sink_in = sink_logit.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
            if sink_in.numel() not in (1, H):
                raise ValueError(f"sink_logit must broadcast to ({H},)")
        ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        q_s = torch.empty_like(q)
        sink = torch.empty(H, dtype=torch.float32, device=dev) if has_sink else None
        flag = torch.empty(1, dtype=torch.int32, device=dev)
        o = torch.empty_like(q)
        stat = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        nsink = sink_in.numel() if has_sink else 0
        if plan.variant == _lib.ATTN_GUARDED:
            # q_s, sink/c, the guard and the guarded forward (flash.py:823-856) in one call.
            _lib.check(lib.alg_attn_fwd_guarded(
                st, dt, plan.layout, B, H, T, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink_in), nsink,
                plan.c, plan.n, _lib.ptr(q_s), _lib.ptr(sink), _lib.ptr(flag), _lib.ptr(o), None, _lib.ptr(stat),
                _lib.ptr(ws), ws_bytes), "flash_attention forward")
        else:
            _lib.check(lib.alg_attn_prepare(
                st, dt, B, H, T, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink_in), nsink, plan.c, plan.n,
                int(plan.range_guard), _lib.ptr(q_s), _lib.ptr(sink), _lib.ptr(flag), _lib.ptr(ws), ws_bytes),
                "flash_attention prologue")
            _lib.check(lib.alg_attn_fwd(
                st, dt, plan.layout, B, H, T, D, _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink), plan.n,
                plan.variant, _lib.ptr(flag), plan.clamp, int(plan.fast_rho), int(plan.inv_stat),
                _lib.ptr(o), None, _lib.ptr(stat)), "flash_attention forward")
        ctx.plan = plan
        ctx.sink_shape = None if not has_sink else tuple(sink_logit.shape)
        ctx.sink_dtype = None if not has_sink else sink_logit.dtype
        ctx.save_for_backward(q_s, k, v, sink, o, stat, flag)
        return o

    @staticmethod
    def backward(ctx, do):
        q_s, k, v, sink, o, stat, flag = ctx.saved_tensors
        plan = ctx.plan
        B, H, T, D = _bhtd(q_s.shape, plan.layout)
        lib = _lib.load()
        dt = _DTYPES[q_s.dtype]
        dev = q_s.device
        st = _lib.stream_of(q_s)
        do = _lib.aligned16(do.to(q_s.dtype))
        ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        dq = torch.empty_like(q_s)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        di = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        dbeta = torch.empty(H, dtype=torch.float32, device=dev) if sink is not None else None
        alpha = 1.0 / (math.sqrt(D) * plan.c)
        _lib.check(lib.alg_attn_bwd(
            st, dt, plan.layout, B, H, T, D, _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink), _lib.ptr(o),
            _lib.ptr(stat), _lib.ptr(do), plan.n, plan.variant, _lib.ptr(flag), plan.clamp,
            int(plan.fast_rho), int(plan.inv_stat), alpha, _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(di),
            _lib.ptr(dbeta), _lib.ptr(ws), ws_bytes), "flash_attention backward")
        dsink = None
        if sink is not None:
            # sink = broadcast(reshape(sink_logit, -1), (H,)) / c  (flash.py:826-828)
            g = dbeta / plan.c
            numel = math.prod(ctx.sink_shape) if ctx.sink_shape else 1
            g = g if numel == H else g.sum().reshape(1)
            dsink = g.reshape(ctx.sink_shape).to(ctx.sink_dtype)
        return dq, dk, dv, dsink, None


def flash_attention(q, k, v, sink_logit=None, *, kind: str = "softmax",
                    n: int = 16, c: float = 16.0, block: int = 512,
                    block_q: Optional[int] = None, block_k: Optional[int] = None,
                    shift: Optional[bool] = None, fast_rho: Optional[bool] = None,
                    inv_stat: Optional[bool] = None, compact_stat: bool = True,
                    poly_rho: bool = False, range_guard: bool = False,
                    resident_bwd: Optional[bool] = None,
                    diagonal_bwd: Optional[bool] = None,
                    diagonal_fwd: Optional[bool] = None,
                    head_resident: Optional[bool] = None, layout: str = "bhtd"):
    """Causal attention on (B, H, T, D) GPU tensors; ``sink_logit`` broadcastable to (H,).

    Same arguments, validation and maths as flash.py:763-857 for ``kind="asinh"``.
    Differentiable in q, k, v and sink_logit through torch autograd.
    ``layout="bthd"`` (an addition to the reference's signature) takes q, k, v in the
    projection layout (B, T, H, D) of model.py:167-169 and returns o in it, so the model's
    head transposes (model.py:167-169, 182) and their copies drop out: ``o.reshape(B, T, H*D)``
    is a view.
    """
    plan = _make_plan(q, k, v, kind, n, c, block, block_q, block_k, shift, fast_rho, inv_stat, compact_stat,
                      poly_rho, range_guard, resident_bwd, diagonal_bwd, diagonal_fwd, head_resident, layout)
    D = q.shape[-1]
    if D in _BUILT_D:
        return _FlashFn.apply(q, k, v, sink_logit, plan)
    return _padded(q, k, v, sink_logit, plan, D)


# Head widths the gfx950 kernels are built for. The reference's generic kernels take any D
# (flash.py:189-326); other widths up to 128 run here on the next built width with zero
# columns appended to q, k and v: a zero column adds nothing to any q.k product, so the
# scores, weights and row statistics are those of the unpadded call, the padded columns of
# o, dq, dk and dv come out exactly zero, and they are dropped. Two scalars must see the
# logical width: alpha = 1/(sqrt(D) c) (flash.py:823) and sink/c. The padded call therefore
# runs with c' = c sqrt(D / Dp), whose alpha 1/(sqrt(Dp) c') is the reference's, and with the
# sink scaled by c'/c so that sink'/c' = sink/c; the gradients flow back through the
# padding, the slice and that scaling. The C ABI itself takes D in {64, 128}.
_BUILT_D = (64, 128)


def _padded(q, k, v, sink_logit, plan, D):
    Dp = next(w for w in _BUILT_D if w >= D)
    c_pad = plan.c * math.sqrt(D / Dp)
    pad = lambda t: torch.nn.functional.pad(t, (0, Dp - D))
    sink_pad = None if sink_logit is None else sink_logit * (c_pad / plan.c)
    o = _FlashFn.apply(pad(q), pad(k), pad(v), sink_pad, plan._replace(c=c_pad))
    return o[..., :D].contiguous()


_LAYOUTS = {"bhtd": 0, "bthd": 1}


def _bhtd(shape, layout: int):
    """(B, H, T, D) of a tensor stored in `layout`."""
    if layout == _lib.LAYOUT_BTHD:
        B, T, H, D = shape
        return B, H, T, D
    return tuple(shape)


def _make_plan(q, k, v, kind, n, c, block, block_q, block_k, shift, fast_rho, inv_stat, compact_stat, poly_rho,
               range_guard, resident_bwd, diagonal_bwd, diagonal_fwd, head_resident, layout="bhtd") -> _Plan:
    """Argument validation of flash.py:793-822 and the kernel variant it selects."""
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}")
    lay = _LAYOUTS[layout]
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must share the shape " + ("(B, T, H, D)" if lay else "(B, H, T, D)"))
    B, H, T, D = _bhtd(q.shape, lay)
    bq = min(block_q or block, T)
    bk = min(block_k or block, T)
    if T % bq or T % bk:
        raise ValueError(f"sequence length {T} must be divisible by blocks ({bq}, {bk})")
    var = make_variant(kind, n, c, T, shift, fast_rho, inv_stat, compact_stat, poly_rho)
    # Schedule-knob validation of flash.py:799-820 (the knobs do not change the maths).
    resident_supported = (T in (512, 1024, 2048) and D == 64 and
                          q.dtype == k.dtype == v.dtype == torch.bfloat16 and not poly_rho and
                          (kind == "softmax" or n == 16))
    if resident_bwd is True and not resident_supported:
        raise ValueError("resident backward needs bfloat16, T=512/1024/2048, D=64, "
                         "and softmax or exact asinh n=16")
    use_resident = (resident_supported and T == 2048 and bq == bk == 512 and compact_stat
                    if resident_bwd is None else bool(resident_bwd))
    if diagonal_bwd is True and not use_resident:
        raise ValueError("diagonal backward requires the resident backward backend")
    head_supported = (use_resident and T == 2048 and bq == bk == 512 and compact_stat)
    if head_resident is True and not head_supported:
        raise ValueError("whole-head residency needs resident bfloat16 T=2048,D=64, "
                         "512-square public tiles, and compact statistics")
    if kind == "softmax":
        raise NotImplementedError("kind='softmax' is the transcendental control arm; only the "
                                  "algebraic kind='asinh' path is built for MI355X")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise NotImplementedError(f"dtype {q.dtype}: gfx950 kernels take bfloat16 or float32 inputs")
    if range_guard and kind == "asinh" and n <= 32:
        if poly_rho:
            raise ValueError("range_guard is for exact radical evaluation")
        plan = _Plan(_lib.ATTN_GUARDED, var.n, float(c), var.clamp, True, True, True, lay)
    else:
        if var.poly_rho:
            raise NotImplementedError("poly_rho is an opt-in TPU experiment; use exact rho")
        if var.shift:
            plan = _Plan(_lib.ATTN_SHIFTED, var.n, float(c), var.clamp, var.fast_rho, False, False, lay)
        else:
            if not var.fast_rho:
                raise NotImplementedError("unshifted accumulation is built with fast rho (the default)")
            plan = _Plan(_lib.ATTN_CLIPPED, var.n, float(c), var.clamp, True, var.inv_stat, False, lay)
    if D > 128:
        raise NotImplementedError(f"head_dim {D}: gfx950 kernels are built for head_dim <= 128")
    if not q.is_cuda:
        raise RuntimeError("flash_attention needs GPU tensors (no CPU fallback)")
    return plan
