"""RMS normalisation with a learned gain on MI355X: the model's final norm ahead of the head.

``rms_norm(x, gain, eps)`` mirrors ``algebraic.rms_norm`` (src/algebraic/algebraic.py:76-83)
as the model uses it before the head (src/algebraic/model.py:208): bfloat16 rows, f32
statistics, one rounding to bfloat16; differentiable in x and the gain, with the VJP JAX's
autodiff forms for that expression. Both passes are HIP kernels (one wave per row); compose
with the head as ``fused_head(rms_norm(x, g), E, t, ...)``. No CPU fallback.
"""

import torch

from .. import _lib


class _RmsNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gain, eps):
        lib = _lib.load()
        d = x.shape[-1]
        x2 = _lib.aligned16(x).reshape(-1, d)
        rows = x2.shape[0]
        g = None if gain is None else gain.detach().to(device=x.device, dtype=torch.float32).contiguous()
        y = torch.empty_like(x2)
        tau = torch.empty(rows, dtype=torch.float32, device=x.device)
        _lib.check(lib.alg_rms_norm_fwd(_lib.stream_of(x2), rows, d, _lib.ptr(x2), _lib.ptr(g), float(eps),
                                        _lib.ptr(y), _lib.ptr(tau)), "rms_norm")
        ctx.save_for_backward(x2, g, tau)
        ctx.gain_meta = None if gain is None else (gain.shape, gain.dtype)
        ctx.shape = x.shape
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, g, tau = ctx.saved_tensors
        lib = _lib.load()
        rows, d = x2.shape
        dy2 = _lib.aligned16(dy.to(x2.dtype)).reshape(rows, d)
        dx = torch.empty_like(x2)
        dg = torch.empty(d, dtype=torch.float32, device=x2.device) if g is not None else None
        nbytes = lib.alg_rms_norm_workspace_size(rows, d)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x2.device)
        _lib.check(lib.alg_rms_norm_bwd(_lib.stream_of(x2), rows, d, _lib.ptr(x2), _lib.ptr(g), _lib.ptr(tau),
                                        _lib.ptr(dy2), _lib.ptr(dx), _lib.ptr(dg), _lib.ptr(ws), nbytes),
                   "rms_norm backward")
        dgain = None if dg is None else dg.reshape(ctx.gain_meta[0]).to(ctx.gain_meta[1])
        return dx.reshape(ctx.shape), dgain, None


def rms_norm(x, gain=None, eps: float = 1e-5):
    """``round((x rsqrt(mean(x^2) + eps)) gain)`` over the last axis of a bfloat16 GPU tensor."""
    if x.dtype != torch.bfloat16:
        raise NotImplementedError(f"dtype {x.dtype}: the gfx950 norm takes bfloat16 rows")
    if gain is not None and gain.numel() != x.shape[-1]:
        raise ValueError(f"gain must have {x.shape[-1]} entries")
    if not x.is_cuda:
        raise RuntimeError("rms_norm needs a GPU tensor (no CPU fallback)")
    return _RmsNormFn.apply(x, gain, float(eps))
