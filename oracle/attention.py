"""Causal algebraic attention, restated in NumPy (test infrastructure, never shipped).

Two restatements of the reference:

``dense_forward`` / ``dense_backward`` (float64)
    The dense oracle ``asinh_power_weights`` + ``asinh_attention``
    (src/algebraic/algebraic.py:186-216): scores in full precision, exact max shift,
    optional sink column; its backward is the closed-form VJP JAX autodiff produces
    for that function in exact arithmetic (softmax VJP on the compressed logits
    ``n asinh(s/c)``, paper/paper.tex:443-459).
    Pin: tests/test_oracle.py compares the forward with softmax of ``n*arcsinh(s/c)``
    (tests/test_components.py:27-40 pattern) and the backward with torch float64 autograd
    of that closed form.

``kernel_forward`` / ``kernel_backward`` (float32, cast-faithful)
    The Pallas kernel semantics the HIP kernels replace, with the same rounding points:
    prologue ``q_s = round(q*alpha)`` and ``sink/c`` (flash.py:823-833); in-range
    unshifted forward with fast rho, f32 row sums of unrounded weights and rounded
    weights into PV (flash.py:189-234, 271-284; head_resident.py:25-89); backward tile
    gradients (flash.py:333-361), ``di`` from the rounded output (flash.py:633),
    slope n applied once (flash.py:591-597), sink VJP (flash.py:694-726), and the
    chain rule through ``q_s`` back to ``q``. ``shifted=True`` restates the guarded
    fallback (flash.py:235-259, 280, 347-350, 851-852): max-shifted stable rho,
    ``stat = rho(-m) Z^(-1/n)``, precise (f32) output; for bf16 the backward's ``di`` is
    ``sum_j p_ij dP_ij`` from the f32 weights, as the HIP fallback forms it (it keeps no f32
    copy of the output), instead of ``<dO_i, o_i>`` over that copy.
    Pin: equal to the dense float64 oracle within the bf16/fp32 tolerances
    (tests/test_oracle.py), and to its own float64 evaluation.

``guard_in_range``
    The range-guard predicate (flash.py:834-849).
"""

import math

import numpy as np

from .numerics import attn_clamp, int_pow, inv_root, rho_exact, rho_fast, round_to

F64 = np.float64
F32 = np.float32


def _sink_vector(sink_logit, H):
    """Broadcast ``sink_logit`` to (H,) as flash.py:826-828 does."""
    s = np.asarray(sink_logit, F64).reshape(-1)
    return np.broadcast_to(s, (H,)).astype(F64)


# ---------------------------------------------------------------------------
# Dense float64 oracle (algebraic.py:186-216)
# ---------------------------------------------------------------------------

def _dense_probs(q, k, n, c, sink):
    """Per-(b,h) normalised weights and sink mass, float64, exact max shift.

    Returns (P (B,H,T,T), P_sink (B,H,T), x (B,H,T,T)) with x the kernel-unit score.
    Follows asinh_power_weights (algebraic.py:186-204).
    """
    B, H, T, D = q.shape
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(F64), k.astype(F64)) * (1.0 / math.sqrt(D))
    x = s / c
    mask = np.tril(np.ones((T, T), bool))[None, None]
    m = np.max(np.where(mask, x, -1e300), axis=-1, keepdims=True)
    if sink is not None:
        xb = (sink / c)[None, :, None, None]
        m = np.maximum(m, xb)
    shift = _rho_stable64(-m)
    w = np.where(mask, int_pow(_rho_stable64(x) * shift, n), 0.0)
    denom = np.sum(w, axis=-1, keepdims=True)
    if sink is not None:
        wb = int_pow(_rho_stable64(np.broadcast_to(xb, m.shape)) * shift, n)
        denom = denom + wb
        psink = (wb / denom)[..., 0]
    else:
        psink = np.zeros((B, H, T))
    return w / denom, psink, x


def _rho_stable64(x):
    x = np.asarray(x, F64)
    rad = 1.0 + x * x
    t = np.abs(x) + np.sqrt(rad)
    return np.where(x >= 0, t, 1.0 / t)


def dense_forward(q, k, v, sink_logit=None, *, n=16, c=8.0):
    """Dense causal asinh-power attention in float64 (algebraic.py:207-216)."""
    H = q.shape[1]
    sink = None if sink_logit is None else _sink_vector(sink_logit, H)
    p, _, _ = _dense_probs(q, k, n, c, sink)
    return np.einsum("bhqk,bhkd->bhqd", p, v.astype(F64))


def dense_backward(q, k, v, sink_logit, do, *, n=16, c=8.0):
    """Exact-arithmetic VJP of ``dense_forward`` w.r.t. (q, k, v, sink_logit), float64.

    With logits a_ij = n asinh(x_ij), x = s/c, s = q.k/sqrt(D), and the sink a column
    with zero value: dA = P (dP - D_i), D_i = <dO_i, o_i>; dx = n r(x) dA; ds = dx / c;
    dq = ds k / sqrt(D); dk = ds^T q / sqrt(D); dv = P^T dO; d sink_h = sum over rows of
    -P_sink D_i n r(x_b) / c.
    """
    B, H, T, D = q.shape
    sink = None if sink_logit is None else _sink_vector(sink_logit, H)
    q64, k64, v64, do64 = (a.astype(F64) for a in (q, k, v, do))
    p, psink, x = _dense_probs(q64, k64, n, c, sink)
    o = np.einsum("bhqk,bhkd->bhqd", p, v64)
    dP = np.einsum("bhqd,bhkd->bhqk", do64, v64)
    Di = np.sum(do64 * o, axis=-1, keepdims=True)
    dA = p * (dP - Di)
    r = 1.0 / np.sqrt(1.0 + x * x)
    ds = dA * n * r / c / math.sqrt(D)
    dq = np.einsum("bhqk,bhkd->bhqd", ds, k64)
    dk = np.einsum("bhqk,bhqd->bhkd", ds, q64)
    dv = np.einsum("bhqk,bhqd->bhkd", p, do64)
    dsink = None
    if sink is not None:
        xb = sink / c
        rb = 1.0 / np.sqrt(1.0 + xb * xb)
        dAb = -psink * Di[..., 0]                       # (B,H,T)
        dsink_h = np.sum(dAb, axis=(0, 2)) * n * rb / c  # (H,)
        shape = np.shape(sink_logit)
        size = int(np.prod(shape)) if len(shape) else 1
        dsink = dsink_h.reshape(-1) if size == H else np.array([dsink_h.sum()])
        dsink = dsink.reshape(shape)
    return dq, dk, dv, dsink


# ---------------------------------------------------------------------------
# Range guard (flash.py:834-849)
# ---------------------------------------------------------------------------

def guard_in_range(q_s, k, v, sink, *, n=16, has_sink=True):
    """Runtime predicate choosing the unshifted branch; ``sink`` already divided by c."""
    T = q_s.shape[2]
    bound = min(16.0, attn_clamp(T, n) / 2)
    q2 = np.max(np.sum(q_s.astype(F32) ** 2, axis=-1))
    k2 = np.max(np.sum(k.astype(F32) ** 2, axis=-1))
    ok = bool(np.float32(q2) * np.float32(k2) <= (bound / 1.01) ** 2)
    if has_sink:
        ok = ok and bool(np.max(np.abs(sink)) <= bound / 1.01)
    vmax = min(1e8, 1e37 / ((T + int(has_sink)) * (2 * bound + 1) ** n))
    ok = ok and bool(np.max(np.abs(v.astype(F32))) <= vmax)
    return ok


# ---------------------------------------------------------------------------
# Cast-faithful kernel restatement (flash.py / head_resident.py)
# ---------------------------------------------------------------------------

def prologue(q, sink_logit, *, c=8.0, dtype="bf16"):
    """``q_s = round(q*alpha)`` with alpha = 1/(sqrt(D) c), and ``sink/c`` (flash.py:823-833)."""
    B, H, T, D = q.shape
    alpha = 1.0 / (math.sqrt(D) * float(c))
    q_s = round_to(q.astype(F32) * F32(alpha), dtype)
    sink = None if sink_logit is None else (_sink_vector(sink_logit, H) / c).astype(F32)
    return q_s, sink, alpha


def kernel_forward(q_s, k, v, sink, *, n=16, dtype="bf16", shifted=False, heads=None, rows=None):
    """Forward of the kernel on pre-scaled queries; returns (o, stat, o_precise).

    Unshifted (in range): w = rho_fast(x)^n, Z = rho_fast(beta)^n + sum_j w,
    o = round(sum_j round(w) v * (1/Z)), stat = 1/Z (flash.py:197-234, 271-284).
    Shifted fallback: m = max(beta, max_j x); w = (rho(x) rho(-m))^n with stable rho;
    stat = rho(-m) Z^(-1/n); o kept in f32 as well (precise_output).
    ``heads`` restricts the computation to a list of (b, h) pairs and ``rows`` to a list of
    query rows (each row still sees every causal key j <= i); entries outside them stay 0.
    Both bound the CPU work at long sequence lengths.
    """
    B, H, T, D = q_s.shape
    o = np.zeros((B, H, T, D), F32)
    o_precise = np.zeros((B, H, T, D), F32)
    stat = np.zeros((B, H, T), F32)
    ri = np.arange(T) if rows is None else np.asarray(rows)
    mask = ri[:, None] >= np.arange(T)[None, :]
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    for b, h in pairs:
        qb = q_s[b, h][ri].astype(F32)
        kb = k[b, h].astype(F32)
        vb = v[b, h].astype(F32)
        x = qb @ kb.T
        if not shifted:
            w = np.where(mask, int_pow(rho_fast(x)[0], n), F32(0)).astype(F32)
            Z = np.sum(w, axis=1, dtype=F32)
            if sink is not None:
                Z = Z + int_pow(rho_fast(F32(sink[h]))[0], n)
            acc = round_to(w, dtype) @ vb
            inv = (F32(1) / Z).astype(F32)
            o[b, h, ri] = round_to(acc * inv[:, None], dtype)
            o_precise[b, h, ri] = acc * inv[:, None]
            stat[b, h, ri] = inv
        else:
            xm = np.where(mask, x, -np.inf)
            m = np.max(xm, axis=1)
            if sink is not None:
                m = np.maximum(m, F32(sink[h]))
            shift = rho_exact(-m)[0].astype(F32)
            w = np.where(mask, int_pow(rho_exact(np.where(mask, x, 0))[0] * shift[:, None], n), 0).astype(F32)
            Z = np.sum(w, axis=1, dtype=F32)
            if sink is not None:
                Z = Z + int_pow(rho_exact(F32(sink[h]))[0] * shift, n)
            acc = round_to(w, dtype) @ vb
            inv = (F32(1) / Z).astype(F32)
            o_precise[b, h, ri] = acc * inv[:, None]
            o[b, h, ri] = round_to(o_precise[b, h, ri], dtype)
            stat[b, h, ri] = shift * inv_root(Z, n)
    return o, stat, o_precise


def kernel_backward(q_s, k, v, sink, o, stat, do, *, n=16, alpha=None, dtype="bf16",
                    shifted=False, heads=None, di_from_weights=False):
    """Backward of the kernel; returns (dq_s, dk, dv, di, dbeta[, dq]).

    Per tile (flash.py:333-361): p = rho^n * stat (in range, inv_stat) or (rho*stat)^n
    (shifted); dp = dO v^T; ds = p (dp - di) r. dV = round(p)^T dO; dK = n round(ds)^T q_s;
    dq_s = n round(ds) k (flash.py:573-597). di = sum(dO*o) from the given ``o``
    (flash.py:633, 715), or with ``di_from_weights`` di = sum_j p_ij dp_ij from the f32
    weights (the HIP bf16 shifted fallback, which keeps no f32 copy of its output; the two
    agree in exact arithmetic, and this one makes sum_j p_ij (dp_ij - di_i) vanish).
    dbeta_h = -sum_{b,t} mass*di * n r(beta) with mass = rho(beta)^n stat (in range) or
    (rho(beta) stat)^n (shifted), rho stable (flash.py:694-705, 721-723).
    If ``alpha`` is given also returns dq = round(dq_s * alpha) (chain rule through q_s).
    """
    B, H, T, D = q_s.shape
    dq_s = np.zeros((B, H, T, D), F32)
    dk = np.zeros((B, H, T, D), F32)
    dv = np.zeros((B, H, T, D), F32)
    di = np.sum(do.astype(F32) * o.astype(F32), axis=-1, dtype=F32)
    if di_from_weights:
        di = np.zeros((B, H, T), F32)
    mask = np.tril(np.ones((T, T), bool))
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    for b, h in pairs:
        qb, kb, vb, dob = (a[b, h].astype(F32) for a in (q_s, k, v, do))
        st = stat[b, h][:, None]
        x = qb @ kb.T
        if not shifted:
            rho, r = rho_fast(x)
            p = np.where(mask, int_pow(rho, n) * st, F32(0))
        else:
            rho, r = rho_exact(np.where(mask, x, 0))
            p = np.where(mask, int_pow(rho * st, n), F32(0))
        p = p.astype(F32)
        dp = dob @ vb.T
        if di_from_weights:
            di[b, h] = np.sum(p * dp, axis=1, dtype=F32)
        ds = (p * (dp - di[b, h][:, None]) * r).astype(F32)
        dsb = round_to(ds, dtype)
        dv[b, h] = round_to(round_to(p, dtype).T @ dob, dtype)
        dk[b, h] = round_to((dsb.T @ qb) * F32(n), dtype)
        dq_s[b, h] = round_to((dsb @ kb) * F32(n), dtype)
    dbeta = np.zeros((H,), F32)
    if sink is not None:
        rb, r_b = rho_exact(sink.astype(F32))
        if not shifted:
            mass = int_pow(rb[None, :, None], n) * stat
        else:
            mass = int_pow(rb[None, :, None] * stat, n)
        slope = F32(n) * r_b
        dbeta = (-np.sum(mass * di, axis=(0, 2)) * slope).astype(F32)
    out = (dq_s, dk, dv, di, dbeta)
    if alpha is not None:
        dq = round_to(dq_s * F32(alpha), dtype)
        out = out + (dq,)
    return out


def flash_attention_oracle(q, k, v, sink_logit, do=None, *, n=16, c=8.0, dtype="bf16", di_rule=None):
    """Full guarded path: prologue, guard, kernel fwd (and bwd when ``do`` is given).

    Returns a dict with o, stat, q_s, in_range and, with ``do``: dq, dk, dv, dsink_logit.
    Mirrors flash_attention(kind="asinh", range_guard=True) (flash.py:763-857).
    ``di_rule`` picks how the shifted fallback's backward forms di: "precise_output" is the
    reference's (di = <dO, o_precise> over the f32 output it keeps, flash.py:73, 322, 852),
    "weights" the HIP bf16 fallback's (di = sum_j p_ij dP_ij, no f32 output kept). The
    default is what the HIP path does: "weights" for bf16, "precise_output" for f32.
    In range both rules read di from the rounded output (flash.py:633).
    """
    if di_rule is None:
        di_rule = "weights" if dtype == "bf16" else "precise_output"
    if di_rule not in ("weights", "precise_output"):
        raise ValueError(f"di_rule {di_rule!r}")
    q_s, sink, alpha = prologue(q, sink_logit, c=c, dtype=dtype)
    ok = guard_in_range(q_s, k, v, sink if sink is not None else np.zeros(1, F32), n=n,
                        has_sink=sink is not None)
    o, stat, o_precise = kernel_forward(q_s, k, v, sink, n=n, dtype=dtype, shifted=not ok)
    res = dict(o=o, stat=stat, q_s=q_s, in_range=ok, o_precise=o_precise)
    if do is not None:
        # In range di comes from the rounded output; on the fallback from the f32 output
        # (the reference) or from the weights (the HIP bf16 kernels).
        o_di = o if ok else o_precise
        dq_s, dk, dv, di, dbeta, dq = kernel_backward(q_s, k, v, sink, o_di, stat, do, n=n, alpha=alpha,
                                                       dtype=dtype, shifted=not ok,
                                                       di_from_weights=di_rule == "weights" and not ok)
        res.update(dq=dq, dk=dk, dv=dv, di=di)
        if sink_logit is not None:
            shape = np.shape(sink_logit)
            size = int(np.prod(shape)) if len(shape) else 1
            dsl = dbeta / F32(c)
            dsl = dsl if size == q.shape[1] else np.array([dsl.sum()], F32)
            res["dsink"] = dsl.reshape(shape)
    return res


def attention_flops(B, H, T, D, fwd_bwd=False):
    """Algorithmic FLOPs: 4 B H T^2 D / 2 causal forward; x3.5 for fwd+bwd
    (scripts/bench_attention.py:50, 65; scripts/benchmark_throughput.py:71, 103)."""
    f = 4.0 * B * H * T * T * D / 2
    return 3.5 * f if fwd_bwd else f
