"""Fused attention prologue on MI355X: QK RMS norm with gain, Cayley rotation and the
attention pre-scale and range guard in one HIP pass, with its VJP in one pass back.

The model's path into the attention kernel (src/algebraic/model.py:170-174, 181) is

    q = rms_norm(q, q_gain, eps); k = rms_norm(k, k_gain, eps)    # algebraic.py:76-83
    q = apply_rotary(q, cos, sin); k = apply_rotary(k, cos, sin)   # algebraic.py:172-179
    o = flash_attention(q, k, v, sink, kind="asinh", n=n, c=c, range_guard=True)

``qk_norm_rotary_flash_attention`` computes the same function, differentiable in q, k, v,
the sink and both gains, with the normalisation, rotation, ``q*alpha`` and the guard's
maxima in one HIP pass (q, k and v read once; q_s and the rotated k written once) and the
VJP of normalisation and rotation in one pass after the attention backward. The Cayley
tables (``cayley_powers``, ``cayley_table_geometric``; algebraic.py:124-169) are built by a
HIP kernel. There is no CPU fallback: the library must be present and tensors on a GPU.
"""

import math
from typing import Optional

import torch

from .. import _lib
from .flash import _DTYPES, _bhtd, _make_plan


def cayley_powers(w: torch.Tensor, seq_len: int):
    """(cos, sin), each (seq_len, len(w)) float32 on w's device (algebraic.py:124-149)."""
    if w.dim() != 1:
        raise ValueError("w must be one-dimensional")
    if not w.is_cuda:
        raise RuntimeError("cayley_powers needs a GPU tensor (no CPU fallback)")
    lib = _lib.load()
    w = w.detach().to(torch.float32).contiguous()
    half = w.numel()
    cos = torch.empty((seq_len, half), dtype=torch.float32, device=w.device)
    sin = torch.empty_like(cos)
    _lib.check(lib.alg_cayley_tables(_lib.stream_of(w), _lib.ptr(w), half, seq_len, _lib.ptr(cos), _lib.ptr(sin)),
               "cayley_powers")
    return cos, sin


def cayley_table_geometric(head_dim: int, seq_len: int, base: float = 10000.0, w0: float = 0.5,
                           fraction: float = 1.0, device="cuda"):
    """Geometric grid w_k = w0 base^(-k/half), partial rotary by ``fraction``
    (algebraic.py:152-169), tables built on ``device``."""
    half = head_dim // 2
    levels = int(round(math.log2(half)))
    if 1 << levels != half:
        raise ValueError("geometric Cayley grid needs head_dim/2 to be a power of two")
    root = float(base)
    for _ in range(levels):
        root = math.sqrt(root)
    ratio = 1.0 / root
    active = int(round(fraction * half))
    w = [w0 * ratio ** i if i < active else 0.0 for i in range(half)]
    return cayley_powers(torch.tensor(w, dtype=torch.float32, device=device), seq_len)


def _f32_or_none(t, dev):
    return None if t is None else t.detach().to(device=dev, dtype=torch.float32).contiguous()


class _PrologueFlashFn(torch.autograd.Function):
    """norm + gain, rotation, flash_attention as one custom VJP over the HIP kernels."""

    @staticmethod
    def forward(ctx, q, k, v, sink_logit, q_gain, k_gain, cos, sin, eps, plan):
        B, H, T, D = _bhtd(q.shape, plan.layout)
        lib = _lib.load()
        dt = _DTYPES[q.dtype]
        dev = q.device
        st = _lib.stream_of(q)
        q, k, v = _lib.aligned16(q), _lib.aligned16(k), _lib.aligned16(v)
        gq, gk = _f32_or_none(q_gain, dev), _f32_or_none(k_gain, dev)
        cs, sn = _f32_or_none(cos, dev), _f32_or_none(sin, dev)
        if cs is not None and (cs.shape[0] < T or cs.shape[1] != D // 2 or sn.shape != cs.shape):
            raise ValueError(f"cos/sin tables must be (>= {T}, {D // 2})")
        if cs is not None and cs.shape[0] != T:
            cs, sn = cs[:T].contiguous(), sn[:T].contiguous()  # cos[:t] (algebraic.py:175-176)
        for name, g in (("q_gain", gq), ("k_gain", gk)):
            if g is not None and g.numel() != D:
                raise ValueError(f"{name} must have {D} entries")
        has_sink = sink_logit is not None
        sink_in = None
        if has_sink:
            sink_in = sink_logit.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
            if sink_in.numel() not in (1, H):
                raise ValueError(f"sink_logit must broadcast to ({H},)")
        ws_bytes = lib.alg_attn_prologue_workspace_size(B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        q_s, k_r = torch.empty_like(q), torch.empty_like(k)
        tau_q = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        tau_k = torch.empty_like(tau_q)
        sink = torch.empty(H, dtype=torch.float32, device=dev) if has_sink else None
        flag = torch.empty(1, dtype=torch.int32, device=dev)
        _lib.check(lib.alg_attn_qk_prologue(
            st, dt, plan.layout, B, H, T, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(gq), _lib.ptr(gk),
            _lib.ptr(cs), _lib.ptr(sn), float(eps), _lib.ptr(sink_in), sink_in.numel() if has_sink else 0, plan.c,
            plan.n, int(plan.range_guard), _lib.ptr(q_s), _lib.ptr(k_r), _lib.ptr(tau_q), _lib.ptr(tau_k),
            _lib.ptr(sink), _lib.ptr(flag), _lib.ptr(ws), ws_bytes), "attention prologue")
        o = torch.empty_like(q)
        stat = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        _lib.check(lib.alg_attn_fwd(
            st, dt, plan.layout, B, H, T, D, _lib.ptr(q_s), _lib.ptr(k_r), _lib.ptr(v), _lib.ptr(sink), plan.n, plan.variant,
            _lib.ptr(flag), plan.clamp, int(plan.fast_rho), int(plan.inv_stat),
            _lib.ptr(o), None, _lib.ptr(stat)), "attention forward")
        ctx.plan = plan
        ctx.sink_shape = None if not has_sink else tuple(sink_logit.shape)
        ctx.sink_dtype = None if not has_sink else sink_logit.dtype
        ctx.gain_meta = [None if g is None else (g.shape, g.dtype) for g in (q_gain, k_gain)]
        ctx.save_for_backward(q, k, v, gq, gk, cs, sn, q_s, k_r, tau_q, tau_k, sink, o, stat, flag)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, gq, gk, cs, sn, q_s, k_r, tau_q, tau_k, sink, o, stat, flag = ctx.saved_tensors
        plan = ctx.plan
        B, H, T, D = _bhtd(q.shape, plan.layout)
        lib = _lib.load()
        dt = _DTYPES[q.dtype]
        dev = q.device
        st = _lib.stream_of(q)
        do = _lib.aligned16(do.to(q.dtype))
        ws_bytes = lib.alg_attn_workspace_size(dt, B, H, T, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        dq_r, dk_r, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        di = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        dbeta = torch.empty(H, dtype=torch.float32, device=dev) if sink is not None else None
        alpha = 1.0 / (math.sqrt(D) * plan.c)
        _lib.check(lib.alg_attn_bwd(
            st, dt, plan.layout, B, H, T, D, _lib.ptr(q_s), _lib.ptr(k_r), _lib.ptr(v), _lib.ptr(sink), _lib.ptr(o),
            _lib.ptr(stat), _lib.ptr(do), plan.n, plan.variant, _lib.ptr(flag), plan.clamp,
            int(plan.fast_rho), int(plan.inv_stat), alpha, _lib.ptr(dq_r), _lib.ptr(dk_r), _lib.ptr(dv),
            _lib.ptr(di), _lib.ptr(dbeta), _lib.ptr(ws), ws_bytes), "attention backward")
        pws_bytes = lib.alg_attn_prologue_workspace_size(B, H, T, D)
        pws = torch.empty(pws_bytes, dtype=torch.uint8, device=dev)
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        dgq = torch.empty(D, dtype=torch.float32, device=dev) if gq is not None else None
        dgk = torch.empty(D, dtype=torch.float32, device=dev) if gk is not None else None
        _lib.check(lib.alg_attn_qk_prologue_bwd(
            st, dt, plan.layout, B, H, T, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(gq), _lib.ptr(gk), _lib.ptr(cs),
            _lib.ptr(sn), _lib.ptr(tau_q), _lib.ptr(tau_k), _lib.ptr(dq_r), _lib.ptr(dk_r), _lib.ptr(dq),
            _lib.ptr(dk), _lib.ptr(dgq), _lib.ptr(dgk), _lib.ptr(pws), pws_bytes), "attention prologue backward")
        dsink = None
        if sink is not None:
            g = dbeta / plan.c
            numel = math.prod(ctx.sink_shape) if ctx.sink_shape else 1
            g = g if numel == H else g.sum().reshape(1)
            dsink = g.reshape(ctx.sink_shape).to(ctx.sink_dtype)
        gains = []
        for dg, meta in zip((dgq, dgk), ctx.gain_meta):
            gains.append(None if meta is None else dg.reshape(meta[0]).to(meta[1]))
        return dq, dk, dv, dsink, gains[0], gains[1], None, None, None, None


def qk_norm_rotary_flash_attention(q, k, v, sink_logit=None, q_gain=None, k_gain=None, cos=None, sin=None, *,
                                   eps: float = 1e-5, kind: str = "asinh", n: int = 16, c: float = 16.0,
                                   block: int = 512, block_q: Optional[int] = None, block_k: Optional[int] = None,
                                   shift: Optional[bool] = None, fast_rho: Optional[bool] = None,
                                   inv_stat: Optional[bool] = None, compact_stat: bool = True,
                                   poly_rho: bool = False, range_guard: bool = False,
                                   resident_bwd: Optional[bool] = None, diagonal_bwd: Optional[bool] = None,
                                   diagonal_fwd: Optional[bool] = None, head_resident: Optional[bool] = None,
                                   layout: str = "bhtd"):
    """``flash_attention(rot(rms_norm(q, q_gain)), rot(rms_norm(k, k_gain)), v, sink, ...)``.

    q, k, v: raw projections (bf16 or f32) on the GPU, (B, H, T, D) or, with
    ``layout="bthd"``, the projection layout (B, T, H, D) (the output then has it too);
    gains (D,) or None; cos/sin: (>= T, D/2) float32 tables or None (no rotation).
    Attention arguments and their validation are flash_attention's (flash.py:763-857).
    Differentiable in q, k, v, sink_logit and the gains.
    """
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin are given together")
    if not (eps > 0) or not math.isfinite(eps):
        raise ValueError("eps must be positive and finite")
    plan = _make_plan(q, k, v, kind, n, c, block, block_q, block_k, shift, fast_rho, inv_stat, compact_stat,
                      poly_rho, range_guard, resident_bwd, diagonal_bwd, diagonal_fwd, head_resident, layout)
    return _PrologueFlashFn.apply(q, k, v, sink_logit, q_gain, k_gain, cos, sin, float(eps), plan)
