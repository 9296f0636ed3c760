"""Fused tied-embedding algebraic likelihood head on MI355X: drop-in for
``algebraic.kernels.fused_head``.

Mirrors ``fused_head(h, embed, targets, *, kind, n, c, block_n, block_v)``
(src/algebraic/kernels/fused_head.py:260-275) and its custom VJP (232-257) over torch
tensors on the GPU. The logits are never materialised: the forward is one tiled
``E h^T`` MFMA pass with the row statistics fused into its epilogue; the backward reads the
forward's bf16 residual, or recomputes the tiles and forms the logit gradient (bf16, or f32
for f32 hidden states) in a workspace, whole or one vocabulary chunk at a time (the
"streamed" schedule, which holds no (N, V) block), and runs the two gradient GEMMs in HIP
(including the embedding gradient the reference leaves to XLA, fused_head.py:215). Returns ``(objective, telemetry)``: the mean target-miss probability
(whose gradient is the exact NLL gradient) and the per-token target probability, which
receives no gradient. ``kind="ce"`` (the softmax control arm) raises NotImplementedError.
"""

import os

import torch

from .. import _lib

# Backward schedule: "residual" keeps the token-major bf16 block U = w r (and l) from the
# forward so the backward runs 3 products; "recompute" keeps only (h, E, targets, stat) as
# the reference does (fused_head.py:244) and recomputes the logits (4 products) into an
# (N, V) logit-gradient block; "streamed" recomputes them one vocabulary chunk of
# VOCAB_CHUNK rows at a time (0: the library's default) and holds no (N, V) block at all.
# f32 hidden states take the recompute (or streamed) schedule, in f32 throughout as the
# reference runs it.
SCHEDULES = ("residual", "recompute", "streamed")
SCHEDULE = os.environ.get("ALGEBRAIC_HEAD_SCHEDULE", "residual")
VOCAB_CHUNK = int(os.environ.get("ALGEBRAIC_HEAD_VOCAB_CHUNK", "0"))

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _root(value, n):
    out = float(value)
    while n > 1:
        out = out ** 0.5
        n //= 2
    return out


class _HeadFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, h, embed, targets, n, c):
        N, d = h.shape
        V = embed.shape[0]
        lib = _lib.load()
        dev = h.device
        st = _lib.stream_of(h)
        h = _lib.aligned16(h)
        e = _lib.aligned16(embed.detach().to(h.dtype))        # fused_head.py:168
        t = targets.to(device=dev, dtype=torch.int32).contiguous()
        dt = _DTYPES[h.dtype]
        if SCHEDULE not in SCHEDULES:
            raise ValueError(f"head schedule {SCHEDULE!r}: one of {SCHEDULES}")
        if SCHEDULE == "streamed" and (VOCAB_CHUNK < 0 or VOCAB_CHUNK % 256):
            raise ValueError(f"vocab chunk {VOCAB_CHUNK}: 0 or a positive multiple of 256")
        ws_bytes = lib.alg_head_workspace_size(dt, N, d, V, 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        stat = torch.empty(N, dtype=torch.float32, device=dev)
        zt = torch.empty(N, dtype=torch.float32, device=dev)
        pt = torch.empty(N, dtype=torch.float32, device=dev)
        obj = torch.empty((), dtype=torch.float32, device=dev)
        residual = None
        # n = 1 takes the recompute schedule: fused_head.py:59-65 forms l^(-1/n) as rsqrt(l)
        # for n = 1 (not 1/l), which the kernels reproduce, and the residual schedule's
        # U' = (l / s) dz needs stat^n = 1/l.
        if SCHEDULE == "residual" and dt == _lib.DTYPE_BF16 and n > 1 and any(ctx.needs_input_grad[:2]):
            residual = torch.empty(lib.alg_head_residual_size(N, d, V), dtype=torch.uint8, device=dev)
        _lib.check(lib.alg_head_fwd(st, dt, N, d, V, _lib.ptr(h), _lib.ptr(e), _lib.ptr(t), n, c, _lib.ptr(stat),
                                    _lib.ptr(zt), _lib.ptr(pt), _lib.ptr(obj), _lib.ptr(residual),
                                    _lib.ptr(ws), ws_bytes),
                   "fused_head forward")
        ctx.n, ctx.c = n, c
        ctx.streamed = SCHEDULE == "streamed"
        ctx.vocab_chunk = VOCAB_CHUNK
        ctx.embed_dtype = embed.dtype
        ctx.save_for_backward(h, e, t, stat, residual)
        ctx.mark_non_differentiable(pt)
        return obj, pt

    @staticmethod
    def backward(ctx, g_obj, g_tel):
        h, e, t, stat, residual = ctx.saved_tensors
        N, d = h.shape
        V = e.shape[0]
        lib = _lib.load()
        dev = h.device
        st = _lib.stream_of(h)
        g = (g_obj if g_obj is not None else torch.zeros((), device=dev)).to(torch.float32).reshape(1).contiguous()
        dt = _DTYPES[h.dtype]
        dh = torch.empty_like(h)
        de_f32 = ctx.embed_dtype == torch.float32
        de_dt = _lib.DTYPE_F32 if de_f32 else _lib.DTYPE_BF16
        dE = torch.empty((V, d), dtype=torch.float32 if de_f32 else torch.bfloat16, device=dev)
        if ctx.streamed:
            ws_bytes = lib.alg_head_streamed_workspace_size(dt, N, d, V, ctx.vocab_chunk)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            _lib.check(lib.alg_head_bwd_streamed(st, dt, N, d, V, _lib.ptr(h), _lib.ptr(e), _lib.ptr(t), _lib.ptr(stat),
                                                 _lib.ptr(g), ctx.n, ctx.c, ctx.vocab_chunk, _lib.ptr(dh), _lib.ptr(dE),
                                                 de_dt, _lib.ptr(ws), ws_bytes),
                       "fused_head backward (streamed)")
            return dh, dE.to(ctx.embed_dtype), None, None, None
        ws_bytes = lib.alg_head_workspace_size(dt, N, d, V, 2 if residual is not None else 1)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.alg_head_bwd(st, dt, N, d, V, _lib.ptr(h), _lib.ptr(e), _lib.ptr(t), _lib.ptr(stat), _lib.ptr(g),
                                    ctx.n, ctx.c, _lib.ptr(residual), _lib.ptr(dh), _lib.ptr(dE), de_dt,
                                    _lib.ptr(ws), ws_bytes),
                   "fused_head backward")
        return dh, dE.to(ctx.embed_dtype), None, None, None


def fused_head(h, embed, targets, *, kind="ce", n=16, c=16.0, block_n=128, block_v=512):
    """Fused tied-embedding projection and likelihood objective (fused_head.py:260-275).

    ``h`` (N, d) bfloat16 or float32 hidden states, ``embed`` (V, d) (cast to ``h``'s dtype
    as fused_head.py:168 does), ``targets`` (N,). Returns ``(objective, telemetry)``; the
    telemetry carries no gradient. ``dh`` comes back in ``h``'s dtype, ``dE`` in ``embed``'s.
    """
    if kind not in ("ce", "alg_ce"):
        raise ValueError(kind)
    if kind == "alg_ce" and (n & (n - 1)):
        raise ValueError("n must be a power of two")
    N = h.shape[0]
    bn = min(block_n, N)
    if N % bn:
        raise ValueError(f"token count {N} must be divisible by block {bn}")
    if kind == "ce":
        raise NotImplementedError("kind='ce' is the softmax control arm; only kind='alg_ce' is built for MI355X")
    if h.dtype not in _DTYPES:
        raise NotImplementedError(f"hidden dtype {h.dtype}: the gfx950 head takes bfloat16 or float32 hidden states")
    if not h.is_cuda:
        raise RuntimeError("fused_head needs GPU tensors (no CPU fallback)")
    obj, tel = _HeadFn.apply(h, embed, targets, int(n), float(c))
    return obj, tel.detach()


@torch.no_grad()
def head_logprob(h, embed, targets, *, head="alg_ce", n=8, c=2.0, argmax=True):
    """Per-token ``log p(target)`` with the vocabulary streamed (no (N, V) logits), and the
    argmax token: the scorer's head (src/algebraic/benchmarking.py:178-188) with
    ``logprob_from_logits`` (src/algebraic/evaluation.py:13-23) for ``head="alg_ce"``.

    ``h`` (N, d) bfloat16 or float32, ``embed`` (V, d), ``targets`` (N,). Returns ``(logprob, argmax)``:
    float32 (N,) and int64 (N,) (``None`` when ``argmax=False``). Forward only.
    """
    if head == "ce":
        raise NotImplementedError("head='ce' is the softmax control arm; only head='alg_ce' is built for MI355X")
    if head != "alg_ce":
        raise ValueError(f"unknown head {head!r}")
    if n & (n - 1):
        raise ValueError("n must be a power of two")
    if h.dtype not in _DTYPES:
        raise NotImplementedError(f"hidden dtype {h.dtype}: the gfx950 head takes bfloat16 or float32 hidden states")
    if not h.is_cuda:
        raise RuntimeError("head_logprob needs GPU tensors (no CPU fallback)")
    lib = _lib.load()
    N, d = h.shape
    V = embed.shape[0]
    h = _lib.aligned16(h)
    E = _lib.aligned16(embed.to(h.dtype))  # the cast of fused_head.py:168
    t = targets.to(device=h.device, dtype=torch.int32).contiguous()
    logprob = torch.empty(N, dtype=torch.float32, device=h.device)
    am = torch.empty(N, dtype=torch.int32, device=h.device) if argmax else None
    dt = _DTYPES[h.dtype]
    nbytes = lib.alg_head_workspace_size(dt, N, d, V, 3)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=h.device)
    _lib.check(lib.alg_head_eval(_lib.stream_of(h), dt, N, d, V, _lib.ptr(h), _lib.ptr(E), _lib.ptr(t), int(n), float(c),
                                 _lib.ptr(logprob), _lib.ptr(am), _lib.ptr(ws), nbytes), "head_logprob")
    return logprob, (am.long() if argmax else None)
