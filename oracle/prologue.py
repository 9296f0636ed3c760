"""Attention prologue, restated in NumPy (test infrastructure, never shipped).

The model's path into the attention kernel (src/algebraic/model.py:167-174, 181):
QK RMS normalisation with a learned gain, the geometric Cayley rotation, then inside
flash_attention the query pre-scale ``q_s = round(q * alpha)`` (flash.py:823-833).

``rms_norm``        src/algebraic/algebraic.py:76-83 with the float32 promotion of ``_acc``
                    (25-28): tau = rsqrt(mean(x^2) + eps), y = round((x tau) g).
``cayley_powers``   src/algebraic/algebraic.py:124-149: rows ((1 + i w)^2 / (1 + w^2))^m by
                    binary exponentiation with a renormalisation after every squaring.
``cayley_table_geometric``  algebraic.py:152-169 (w_k = w0 base^(-k/half), roots by repeated
                    square roots, partial rotary by ``fraction``).
``rotary``          algebraic.py:172-179: rotate-half by the tables cast to the input dtype;
                    every bfloat16 product and sum is rounded (XLA evaluates bf16 elementwise
                    ops in float32 and rounds each result).
``prologue_forward``  q_s = round(rot(norm(q, g_q)) alpha), k_r = rot(norm(k, g_k)).
``rotary_vjp`` / ``rms_norm_vjp`` / ``prologue_backward``  the VJPs JAX's autodiff forms for
                    those ops: the rotation's transpose with the same bf16 rounding per product
                    and sum; the RMS-norm VJP in float32,
                    dx = tau g dy - x tau^3 sum(g dy x) / D, dgain = sum_rows dy x tau,
                    rounded to the input dtype once.

Pins (tests/test_prologue_oracle.py): the Cayley tables against cos/sin(2 m atan w)
(tests/test_components.py:59-68) and c^2 + s^2 = 1; the float32 RMS norm and rotation against
float64 closed forms (rotation = complex multiplication, norms preserved); both VJPs and the
whole prologue + dense attention chain against torch float64 autograd; planted mistakes
(dropped gain term, transposed rotation sign) fail those pins.
"""

import math

import numpy as np

from .numerics import round_to

F32 = np.float32
F64 = np.float64


def cayley_powers(w, seq_len):
    """(cos, sin) of shape (seq_len, len(w)), float32, following algebraic.py:124-149."""
    w = np.asarray(w, F32)
    w2 = w * w
    c = ((F32(1) - w2) / (F32(1) + w2)).astype(F32)
    s = ((F32(2) * w) / (F32(1) + w2)).astype(F32)
    pos = np.arange(seq_len, dtype=np.int64)
    out_c = np.ones((seq_len, w.shape[0]), F32)
    out_s = np.zeros((seq_len, w.shape[0]), F32)
    bit = 0
    while (1 << bit) < seq_len:
        take = ((pos >> bit) & 1).astype(bool)[:, None]
        new_c = out_c * c - out_s * s
        new_s = out_c * s + out_s * c
        out_c = np.where(take, new_c, out_c).astype(F32)
        out_s = np.where(take, new_s, out_s).astype(F32)
        c, s = (c * c - s * s).astype(F32), (F32(2) * c * s).astype(F32)
        inv = (F32(1) / np.sqrt(c * c + s * s)).astype(F32)
        c, s = c * inv, s * inv
        bit += 1
    inv = (F32(1) / np.sqrt(out_c * out_c + out_s * out_s)).astype(F32)
    return (out_c * inv).astype(F32), (out_s * inv).astype(F32)


def geometric_frequencies(head_dim, base=10000.0, w0=0.5, fraction=1.0):
    """w_k = w0 base^(-k/half) for the first fraction*half entries, 0 after (algebraic.py:152-168)."""
    half = head_dim // 2
    levels = int(round(math.log2(half)))
    if 1 << levels != half:
        raise ValueError("geometric Cayley grid needs head_dim/2 to be a power of two")
    root = float(base)
    for _ in range(levels):
        root = math.sqrt(root)
    ratio = 1.0 / root
    active = int(round(fraction * half))
    return np.array([w0 * ratio ** i if i < active else 0.0 for i in range(half)], F32)


def cayley_table_geometric(head_dim, seq_len, base=10000.0, w0=0.5, fraction=1.0):
    return cayley_powers(geometric_frequencies(head_dim, base, w0, fraction), seq_len)


def rms_norm(x, gain, eps=1e-5, dtype="bf16"):
    """(y, tau): y = round((x tau) g) over the last axis, tau = rsqrt(mean(x^2) + eps) (f32)."""
    xf = np.asarray(x, F32)
    D = xf.shape[-1]
    ms = (np.sum(xf * xf, axis=-1, dtype=F32) / F32(D)).astype(F32)
    tau = (F32(1) / np.sqrt(ms + F32(eps))).astype(F32)
    y = (xf * tau[..., None]).astype(F32)
    if gain is not None:
        y = (y * np.asarray(gain, F32)).astype(F32)
    return round_to(y, dtype), tau


def _tables(cos, sin, T, dtype):
    return round_to(np.asarray(cos, F32)[:T], dtype), round_to(np.asarray(sin, F32)[:T], dtype)


def rotary(x, cos, sin, dtype="bf16"):
    """Rotate-half of (..., T, D) with per-op rounding to ``dtype`` (algebraic.py:172-179)."""
    half = x.shape[-1] // 2
    c, s = _tables(cos, sin, x.shape[-2], dtype)
    x1, x2 = x[..., :half].astype(F32), x[..., half:].astype(F32)
    r = lambda a: round_to(a, dtype)
    y1 = r(r(x1 * c) - r(x2 * s))
    y2 = r(r(x1 * s) + r(x2 * c))
    return np.concatenate([y1, y2], axis=-1)


def rotary_vjp(dy, cos, sin, dtype="bf16"):
    """Transpose of ``rotary``: dx1 = dy1 c + dy2 s, dx2 = dy2 c - dy1 s, rounded per op."""
    half = dy.shape[-1] // 2
    c, s = _tables(cos, sin, dy.shape[-2], dtype)
    d1, d2 = dy[..., :half].astype(F32), dy[..., half:].astype(F32)
    r = lambda a: round_to(a, dtype)
    dx1 = r(r(d1 * c) + r(d2 * s))
    dx2 = r(r(d2 * c) - r(d1 * s))
    return np.concatenate([dx1, dx2], axis=-1)


def rms_norm_vjp(x, gain, tau, dy, dtype="bf16"):
    """(dx, dgain) of ``rms_norm`` for the cotangent ``dy`` of its rounded output.

    dgain = sum over all leading axes of dy x tau; dx = tau g dy - x tau^3 sum_d(g dy x) / D,
    float32, rounded to ``dtype``.
    """
    xf = np.asarray(x, F32)
    dyf = np.asarray(dy, F32)
    D = xf.shape[-1]
    t = np.asarray(tau, F32)[..., None]
    g = np.ones(D, F32) if gain is None else np.asarray(gain, F32)
    yf = (xf * t).astype(F32)
    dgain = np.sum((dyf * yf).reshape(-1, D), axis=0, dtype=F32)
    a = (g * dyf).astype(F32)
    sa = np.sum(a * xf, axis=-1, dtype=F32)[..., None]
    dxf = (a * t - xf * (t * t * t * sa / F32(D))).astype(F32)
    return round_to(dxf, dtype), dgain


def prologue_forward(q, k, q_gain, k_gain, cos, sin, *, eps=1e-5, c=8.0, dtype="bf16"):
    """(q_s, k_r, q_r, tau_q, tau_k) with q_r = rot(norm(q)), q_s = round(q_r alpha)."""
    D = q.shape[-1]
    alpha = 1.0 / (math.sqrt(D) * float(c))
    qn, tau_q = rms_norm(q, q_gain, eps, dtype)
    kn, tau_k = rms_norm(k, k_gain, eps, dtype)
    q_r = qn if cos is None else rotary(qn, cos, sin, dtype)
    k_r = kn if cos is None else rotary(kn, cos, sin, dtype)
    q_s = round_to(q_r.astype(F32) * F32(alpha), dtype)
    return q_s, k_r, q_r, tau_q, tau_k


def prologue_backward(q, k, q_gain, k_gain, cos, sin, tau_q, tau_k, dq_r, dk_r, *, dtype="bf16"):
    """(dq, dk, dq_gain, dk_gain) from the gradients w.r.t. the rotated q_r and k_r."""
    dqn = dq_r if cos is None else rotary_vjp(dq_r, cos, sin, dtype)
    dkn = dk_r if cos is None else rotary_vjp(dk_r, cos, sin, dtype)
    dq, dgq = rms_norm_vjp(q, q_gain, tau_q, dqn, dtype)
    dk, dgk = rms_norm_vjp(k, k_gain, tau_k, dkn, dtype)
    return dq, dk, dgq, dgk
