"""Scalar building blocks of the algebraic path, restated in NumPy (test infrastructure).

References (``/root/reference``):
* ``rho``          src/algebraic/algebraic.py:31-35 and kernels/flash.py:76-80 (stable form)
* ``rho_fast``     src/algebraic/kernels/flash.py:83-88 (``fast_rho=True`` form)
* ``int_pow``      src/algebraic/algebraic.py:38-51, kernels/flash.py:95-104
* ``inv_root``     src/algebraic/kernels/flash.py:107-114, kernels/fused_head.py:59-65
* ``root``         src/algebraic/kernels/flash.py:117-123
* ``attn_clamp``   src/algebraic/kernels/flash.py:744-748 (make_variant)
* ``head_clamp``   src/algebraic/algebraic.py:277-283, kernels/fused_head.py:273

Pins (tests/test_oracle.py): rho == exp(asinh x) and rho(x) rho(-x) == 1 and the group law
(test_components.py:18-24); int_pow == x**n; inv_root == l**(-1/n); bf16 rounding against
torch's bfloat16 cast.
"""

import math

import numpy as np


def rho(x):
    """Stable ``x + sqrt(1+x^2)``: reciprocal form for negative x (algebraic.py:31-35)."""
    x = np.asarray(x)
    rad = 1.0 + x * x
    t = np.abs(x) + rad / np.sqrt(rad)
    return np.where(x >= 0, t, 1.0 / t)


def rho_fast(x):
    """Fast form ``x + (1+x^2) rsqrt(1+x^2)`` and ``r = rsqrt(1+x^2)`` (flash.py:83-88)."""
    x = np.asarray(x)
    rad = 1.0 + x * x
    r = 1.0 / np.sqrt(rad)
    return x + rad * r, r


def rho_exact(x):
    """Stable rho together with ``r = rsqrt(1+x^2)`` (flash.py:76-80)."""
    x = np.asarray(x)
    rad = 1.0 + x * x
    r = 1.0 / np.sqrt(rad)
    t = np.abs(x) + rad * r
    return np.where(x >= 0, t, 1.0 / t), r


def int_pow(x, n):
    """``x**n`` by binary exponentiation for a static positive integer (algebraic.py:38-51)."""
    n = int(n)
    if n < 1:
        raise ValueError("n must be a positive integer")
    out = None
    base = x
    while n:
        if n & 1:
            out = base if out is None else out * base
        n >>= 1
        if n:
            base = base * base
    return out


def inv_root(l, n):
    """``l**(-1/n)`` for n a power of two: rsqrt then repeated ``y*rsqrt(y)`` (flash.py:107-114)."""
    y = 1.0 / np.sqrt(l)
    k = n // 2
    while k > 1:
        y = y / np.sqrt(y)
        k //= 2
    return y


def root(value, n):
    """``value**(1/n)`` for n a power of two by repeated square roots (flash.py:117-123)."""
    out = float(value)
    while n > 1:
        out = math.sqrt(out)
        n //= 2
    return out


def attn_clamp(seq_len, n):
    """Positive-score clamp of the unshifted attention variant (flash.py:744-748)."""
    t = root(1e37 / (seq_len + 1), n)
    return 0.5 * (t - 1.0 / t)


def head_clamp(vocab, n):
    """Kernel-argument clamp X of the lean likelihood (algebraic.py:277-283, fused_head.py:273)."""
    return 0.25 * root(1e38 / vocab, n)


def round_bf16(x):
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32.

    This is the rounding of ``astype(jnp.bfloat16)`` at every cast point of the reference.
    """
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    u = x.view(np.uint32)
    # u + 0x7FFF + lsb stays below 2^32 for every non-NaN pattern (the largest, -inf, is
    # 0xFF800000); NaN patterns may wrap and are restored below.
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = x[nan]
    return out


def round_to(x, dtype):
    """Cast-faithful rounding to the storage dtype name ('bf16' or 'f32')."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f32":
        return np.asarray(x, np.float32)
    raise ValueError(dtype)


def bf16_bits(x):
    """uint16 bit patterns of float32 values that are exactly bf16-representable."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits):
    bits = np.ascontiguousarray(np.asarray(bits, np.uint16))
    return (bits.astype(np.uint32) << 16).view(np.float32)
