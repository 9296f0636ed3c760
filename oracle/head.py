"""Fused tied-embedding algebraic likelihood head, restated in NumPy (test infrastructure).

``dense_forward`` / ``dense_backward`` (float64)
    The dense branch of ``model.head_loss`` (src/algebraic/model.py:225-230): logits
    ``h E^T`` then the lean likelihood ``algebraic_likelihood_lean`` and its custom VJP
    (src/algebraic/algebraic.py:277-319): x = min(z/c, X), w = (x + sqrt(1+x^2))^n,
    pt = w_t / sum w, obj = mean(1 - pt); gradient g (n/c)/N r (p - y), then the two
    matmul VJPs.
    Pin: tests/test_oracle.py checks the gradient against torch float64 autograd of the
    true NLL ``-mean log softmax(n asinh(z/c))_t`` (tests/test_components.py:43-56,
    src/algebraic/evaluation.py:13-23) and ``pt`` against the same closed form.

``eval_logprob`` (float64)
    The scorer's per-token log-probability and argmax (src/algebraic/evaluation.py:13-23,
    src/algebraic/benchmarking.py:178-188). Pin: tests/test_oracle.py checks it against the log
    of the lean likelihood's pt (tests/test_components.py:56) and a brute-force loop.

``kernel_forward`` / ``kernel_backward`` (float32, cast-faithful)
    The Pallas fused head (src/algebraic/kernels/fused_head.py): E cast to h's dtype
    (168), z in f32, x = min(z * (1/c), X) (98), w = (x + rad rsqrt(rad))^n (99-100),
    l = sum w, stat = l^(-1/n) by rsqrt chain (116), zt (87); telemetry pt with stable rho
    (219-229); backward scale s = g (n/c)/N (251), p = ((x + rad r) stat)^n, dz = (p-y) r,
    dz rounded to bf16 after scaling (145), dh = round(dz E) (147, 254),
    dE = round(dz^T h) in E's dtype (215, 254).
    Pin: equal to the dense float64 oracle within tolerance (tests/test_oracle.py).
"""

import numpy as np

from .numerics import head_clamp, int_pow, inv_root, rho_exact, round_to

F64 = np.float64
F32 = np.float32


def dense_forward(h, E, targets, *, n=8, c=2.0):
    """(obj, pt) of the lean likelihood on float64 logits (algebraic.py:294-301)."""
    z = h.astype(F64) @ E.astype(F64).T
    X = head_clamp(z.shape[-1], n)
    x = np.minimum(z / c, X)
    w = int_pow(x + np.sqrt(1.0 + x * x), n)
    wt = w[np.arange(z.shape[0]), targets]
    pt = wt / np.sum(w, axis=-1)
    return np.mean(1.0 - pt), pt


def dense_backward(h, E, targets, g=1.0, *, n=8, c=2.0):
    """(dh, dE) of the lean custom VJP (algebraic.py:309-316) through z = h E^T, float64."""
    h64, E64 = h.astype(F64), E.astype(F64)
    z = h64 @ E64.T
    N, V = z.shape
    X = head_clamp(V, n)
    x = np.minimum(z / c, X)
    rad = 1.0 + x * x
    r = 1.0 / np.sqrt(rad)
    w = int_pow(x + rad * r, n)
    p = w / np.sum(w, axis=-1, keepdims=True)
    y = np.zeros_like(p)
    y[np.arange(N), targets] = 1.0
    dz = (g * (n / c) / N) * r * (p - y)
    return dz @ E64, dz.T @ h64


def kernel_forward(h, E, targets, *, n=8, c=2.0, dtype="bf16", rows=None, chunk=2048):
    """Per-token (stat, zt) and telemetry (pt, obj) of the fused head forward.

    ``rows`` restricts to a token subset (bounded CPU samples). Tokens are processed in
    chunks so the (chunk, V) logit block bounds memory.
    """
    Eb = round_to(E, dtype).astype(F32)
    hh = h.astype(F32)
    N = h.shape[0]
    V = E.shape[0]
    X = F32(head_clamp(V, n))
    inv_c = F32(1.0 / c)
    idx = np.arange(N) if rows is None else np.asarray(rows)
    stat = np.zeros(N, F32)
    zt = np.zeros(N, F32)
    for s in range(0, len(idx), chunk):
        ids = idx[s:s + chunk]
        z = hh[ids] @ Eb.T
        x = np.minimum(z * inv_c, X)
        rad = F32(1) + x * x
        w = int_pow(x + rad * (F32(1) / np.sqrt(rad)), n)
        stat[ids] = inv_root(np.sum(w, axis=1, dtype=F32), n)
        zt[ids] = z[np.arange(len(ids)), targets[ids]]
    xt = np.minimum(zt / F32(c), X)
    pt = int_pow(rho_exact(xt)[0].astype(F32) * stat, n).astype(F32)
    obj = F32(np.mean(1.0 - pt[idx]))
    return stat, zt, pt, obj


def kernel_backward(h, E, targets, stat, g=1.0, *, n=8, c=2.0, dtype="bf16", e_dtype="bf16",
                    chunk=2048, rows=None, dz_dtype=None):
    """(dh, dE) of the fused head backward with the kernel's rounding points: the logit
    gradient is stored in the hidden dtype (``dzb.astype(dz_ref.dtype)``, fused_head.py:145;
    bf16, or f32 for f32 hidden states), dh in that dtype and dE in ``e_dtype``. ``dz_dtype``
    overrides the logit gradient's storage dtype (the tests plant a wrong rounding with it).

    ``rows`` restricts the work to a token subset (bounded CPU samples): dh is exact on those
    rows (0 elsewhere) and dE then sums only their contributions. The scale keeps the full
    token count N of ``h``.
    """
    Eb = round_to(E, dtype).astype(F32)
    hh = h.astype(F32)
    N = h.shape[0]
    V = E.shape[0]
    X = F32(head_clamp(V, n))
    inv_c = F32(1.0 / c)
    scale = F32(g * (n / c) / N)
    dh = np.zeros(h.shape, F32)
    dE = np.zeros(E.shape, F32)
    idx = np.arange(N) if rows is None else np.asarray(rows)
    for s in range(0, len(idx), chunk):
        ids = idx[s:s + chunk]
        z = hh[ids] @ Eb.T
        x = np.minimum(z * inv_c, X)
        rad = F32(1) + x * x
        r = F32(1) / np.sqrt(rad)
        p = int_pow((x + rad * r) * stat[ids][:, None], n)
        y = np.zeros_like(p)
        y[np.arange(len(ids)), targets[ids]] = 1
        dzb = round_to((p - y) * r * scale, dz_dtype or dtype)
        dh[ids] = dzb @ Eb
        dE += dzb.T @ hh[ids]
    return round_to(dh, dtype), round_to(dE, e_dtype)


def eval_logprob(h, E, targets, *, n=8, c=2.0):
    """(logprob, argmax): log_softmax(n asinh(z/c))[t] on float64 logits
    (src/algebraic/evaluation.py:13-23, head "alg_ce") and argmax of the logits
    (src/algebraic/benchmarking.py:187)."""
    z = h.astype(F64) @ E.astype(F64).T
    a = n * np.arcsinh(z / c)
    m = np.max(a, axis=-1, keepdims=True)
    lse = (m + np.log(np.sum(np.exp(a - m), axis=-1, keepdims=True)))[:, 0]
    lp = a[np.arange(z.shape[0]), targets] - lse
    return lp, np.argmax(z, axis=-1), z


def head_flops(N, d, V):
    """Algorithmic FLOPs of head fwd+bwd: 3 matmuls of 2 N d V (scripts/bench_head.py:35)."""
    return 3.0 * 2.0 * N * d * V
