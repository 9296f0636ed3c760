"""Shared helpers for the parity tests (inputs, tolerances, conversions)."""

import numpy as np

from oracle.numerics import round_bf16


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def rms_norm(x, eps=1e-5):
    """x * rsqrt(mean x^2 + eps) per row (src/algebraic/algebraic.py:76-83, gain 1)."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def attention_inputs(B, H, T, D, *, seed=1, dtype="bf16", qk_norm=True, scale=1.0, sink=True,
                     sink_std=0.1):
    """Q/K/V/dO ~ N(0,1), Q and K RMS-normalised, sink ~ N(0, sink_std) shaped (1,H,1,1)."""
    rng = np.random.default_rng(seed)
    q, k, v, do = (rng.standard_normal((B, H, T, D)).astype(np.float32) for _ in range(4))
    if qk_norm:
        q, k = rms_norm(q), rms_norm(k)
    q, k = q * scale, k * scale
    s = (rng.standard_normal((1, H, 1, 1)) * sink_std).astype(np.float32) if sink else None
    if dtype == "bf16":
        q, k, v, do = (round_bf16(a) for a in (q, k, v, do))
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), do.astype(np.float32), s


def head_inputs(N, d, V, *, seed=2, e_std=0.02):
    """h ~ N(0,1) RMS-normalised (bf16), E ~ N(0, e_std) (bf16), targets uniform."""
    rng = np.random.default_rng(seed)
    h = round_bf16(rms_norm(rng.standard_normal((N, d)).astype(np.float32)))
    E = round_bf16((rng.standard_normal((V, d)) * e_std).astype(np.float32))
    t = rng.integers(0, V, N).astype(np.int32)
    return h, E, t
