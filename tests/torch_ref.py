"""Float32 torch restatement of the kernel semantics, for parity at the BASELINE full sizes.

The NumPy oracle (``oracle/``) is the checker at the sizes it finishes in seconds; at the full
configurations (T = 2048 with 128 heads, T = 16384, N·V = 5e8 logits) the same cast-faithful
formulas are evaluated here with torch on the device the inputs live on, so every output and
gradient of a full-size call can be compared element by element. This module is pinned to the
NumPy oracle by tests/test_torch_ref.py (CPU, small shapes, every output) and, on the GPU, by
the sampled-head / sampled-row comparisons in tests/test_full_size_gpu.py.

Attention (in-range guarded branch, src/algebraic/kernels/flash.py:189-234, 271-284, 333-361,
630-645, 694-729, 823-857): q_s = round(q·alpha), x = q_s·kᵀ (f32), w = rho_fast(x)^n,
Z = rho_fast(beta)^n + sum w (unrounded), o = round(round(w)·v / Z), stat = 1/Z; backward
di = sum dO·o, p = w·stat, ds = p (dO·vᵀ − di) r, dV = round(round(p)ᵀ dO),
dK = round(n round(ds)ᵀ q_s), dq = round(round(n round(ds) k)·alpha),
dbeta = −n r(beta) sum rho_stable(beta)^n stat di.

Head (src/algebraic/kernels/fused_head.py:72-156, 194-275): E cast to h's dtype,
x = min(z/c, X), w = (x + rad rsqrt(rad))^n, stat = l^(-1/n) (rsqrt chain), zt = z[t],
pt = (rho_stable(min(zt/c, X))·stat)^n, obj = mean(1 − pt); backward
dz = round_bf16((p − y) r · g (n/c)/N), dh = round(dz E), dE = round(dz^T h).
"""

import math

import torch

from oracle.numerics import head_clamp

F32 = torch.float32


def _rnd(x, dtype):
    """Round float32 values to the storage dtype (round to nearest even) and back to f32."""
    return x.to(dtype).to(F32) if dtype != F32 else x


def _pow(x, n):
    """x**n for n a power of two by repeated squaring (the kernels' compile-time chain)."""
    while n > 1:
        x = x * x
        n //= 2
    return x


def _rho_fast(x):
    rad = 1.0 + x * x
    r = torch.rsqrt(rad)
    return x + rad * r, r


def _rho_stable(x):
    rad = 1.0 + x * x
    r = torch.rsqrt(rad)
    t = x.abs() + rad * r
    return torch.where(x >= 0, t, 1.0 / t), r


def _inv_root(l, n):
    y = torch.rsqrt(l)
    k = n // 2
    while k > 1:
        y = y * torch.rsqrt(y)
        k //= 2
    return y


def attention(q, k, v, sink_logit, do=None, *, n=16, c=8.0, heads_per_chunk=16):
    """Guarded in-range path on (B,H,T,D) tensors of one dtype (bf16 or f32).

    Returns a dict of float32 tensors: o, stat (and, with ``do``: dq, dk, dv, di, dsink).
    The caller checks that the inputs are in range (the fallback branch is not restated
    here; the NumPy oracle covers it).
    """
    B, H, T, D = q.shape
    dt = q.dtype
    alpha = 1.0 / (math.sqrt(D) * float(c))
    q_s = _rnd(q.to(F32) * alpha, dt)
    kk, vv = k.to(F32), v.to(F32)
    beta = None
    if sink_logit is not None:
        beta = torch.broadcast_to(sink_logit.detach().to(F32).reshape(-1), (H,)) / float(c)
    out = {name: torch.empty((B, H, T, D), dtype=F32, device=q.device) for name in ("o",)}
    out["stat"] = torch.empty((B, H, T), dtype=F32, device=q.device)
    if do is not None:
        for name in ("dq", "dk", "dv"):
            out[name] = torch.empty((B, H, T, D), dtype=F32, device=q.device)
        out["di"] = torch.empty((B, H, T), dtype=F32, device=q.device)
    mask = torch.ones((T, T), dtype=torch.bool, device=q.device).tril()
    flat = [(b, h) for b in range(B) for h in range(H)]
    for s in range(0, len(flat), heads_per_chunk):
        pairs = flat[s:s + heads_per_chunk]
        bi = torch.tensor([p[0] for p in pairs], device=q.device)
        hi = torch.tensor([p[1] for p in pairs], device=q.device)
        qb, kb, vb = q_s[bi, hi], kk[bi, hi], vv[bi, hi]
        x = torch.matmul(qb, kb.transpose(1, 2).contiguous())
        rho, r = _rho_fast(x)
        w = torch.where(mask, _pow(rho, n), torch.zeros((), dtype=F32, device=q.device))
        del rho
        Z = w.sum(-1)
        if beta is not None:
            Z = Z + _pow(_rho_fast(beta[hi])[0], n)[:, None]
        inv = 1.0 / Z
        acc = torch.matmul(_rnd(w, dt), vb)
        o = _rnd(acc * inv[..., None], dt)
        out["o"][bi, hi] = o
        out["stat"][bi, hi] = inv
        if do is None:
            continue
        dob = do[bi, hi].to(F32)
        di = (dob * o).sum(-1)
        p = w * inv[..., None]
        del w
        dp = torch.matmul(dob, vb.transpose(1, 2).contiguous())
        dsb = _rnd(p * (dp - di[..., None]) * r, dt)
        del dp, r
        out["dv"][bi, hi] = _rnd(torch.matmul(_rnd(p, dt).transpose(1, 2).contiguous(), dob), dt)
        out["dk"][bi, hi] = _rnd(torch.matmul(dsb.transpose(1, 2).contiguous(), qb) * float(n), dt)
        dq_s = _rnd(torch.matmul(dsb, kb) * float(n), dt)
        out["dq"][bi, hi] = _rnd(dq_s * alpha, dt)
        out["di"][bi, hi] = di
    if do is not None and beta is not None:
        rb, r_b = _rho_stable(beta)
        mass = _pow(rb[None, :, None], n) * out["stat"]
        dbeta = -(mass * out["di"]).sum(dim=(0, 2)) * (float(n) * r_b)
        out["dsink"] = dbeta / float(c)
    return out


def head(h, E, targets, g=1.0, *, n=8, c=2.0, chunk=4096, backward=True):
    """Fused head forward (and backward for cotangent ``g`` on obj), float32 results.

    Returns a dict: stat, zt, pt, obj (and dh, dE).
    """
    N, d = h.shape
    V = E.shape[0]
    dt = h.dtype
    Eb = E.to(dt).to(F32)
    hh = h.to(F32)
    X = float(head_clamp(V, n))
    inv_c = 1.0 / float(c)
    scale = float(g) * (n / c) / N
    stat = torch.empty(N, dtype=F32, device=h.device)
    zt = torch.empty(N, dtype=F32, device=h.device)
    dh = torch.empty((N, d), dtype=F32, device=h.device) if backward else None
    dE = torch.zeros((V, d), dtype=F32, device=h.device) if backward else None
    tl = targets.to(torch.long)
    for s in range(0, N, chunk):
        ids = slice(s, min(N, s + chunk))
        z = torch.matmul(hh[ids], Eb.t().contiguous())
        rows = torch.arange(z.shape[0], device=h.device)
        zt[ids] = z[rows, tl[ids]]
        x = torch.clamp(z * inv_c, max=X)
        del z
        rad = 1.0 + x * x
        r = torch.rsqrt(rad)
        rho = x + rad * r
        del rad, x
        st = _inv_root(_pow(rho, n).sum(-1), n)
        stat[ids] = st
        if not backward:
            continue
        p = _pow(rho * st[:, None], n)
        p[rows, tl[ids]] -= 1.0
        dzb = _rnd(p * r * scale, torch.bfloat16)
        del p, r, rho
        dh[ids] = torch.matmul(dzb, Eb)
        dE += torch.matmul(dzb.t().contiguous(), hh[ids])
    xt = torch.clamp(zt / float(c), max=X)
    pt = _pow(_rho_stable(xt)[0] * stat, n)
    out = dict(stat=stat, zt=zt, pt=pt, obj=(1.0 - pt).mean())
    if backward:
        out["dh"] = _rnd(dh, dt)
        out["dE"] = _rnd(dE, E.dtype)
    return out
