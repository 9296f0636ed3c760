"""ALU-GLU feed-forward block, restated in NumPy (test infrastructure, never shipped).

``alu_parts`` / ``alu``   src/algebraic/algebraic.py:86-106: bz = beta z, r = rsqrt(1 + bz^2),
                          u = bz r, 1 + u (or r^2/(1 - u) for bz < 0, so the negative tail keeps
                          its precision), alu = round(0.5 z (1 + u)) in x's dtype.
``alu_vjp``               algebraic.py:109-113: g * (0.5 (1 + u) + 0.5 u r^2), rounded to g's dtype.
``ffn_forward`` / ``ffn_backward``  src/algebraic/model.py:185-193 with ffn="alu_glu":
    gate = round(h2 w_g), up = round(h2 w_u), act = alu(up), y = round(gate act),
    out = round(y w_d); backward by JAX's autodiff of those bf16 ops: dy = round(dout w_d^T),
    d_gate = round(dy act), d_act = round(dy gate), d_up = alu_vjp(d_act), then the matmul VJPs
    (f32 accumulation, rounded).

Pins (tests/test_ffn_oracle.py): alu against its closed form x/2 (1 + bx/sqrt(1 + b^2 x^2))
and its VJP against torch float64 autograd of that closed form on [-40, 40]
(tests/test_components.py:71-78), and the whole block's gradients against torch float64
autograd in float32 mode; planted mistakes (the derivative without 0.5 u r^2, gate and up
weights swapped) fail that pin.
"""

import numpy as np

from .numerics import round_to

F32 = np.float32


def alu_parts(x, beta, dtype="bf16"):
    """(alu(x), u, r) with the reference's negative-tail form, f32 arithmetic."""
    z = np.asarray(x, F32)
    bz = (F32(beta) * z).astype(F32)
    r = (F32(1) / np.sqrt(F32(1) + bz * bz)).astype(F32)
    u = (bz * r).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        neg = ((r * r) / (F32(1) - u)).astype(F32)
    one_plus_u = np.where(bz < 0, neg, F32(1) + u).astype(F32)
    return round_to((F32(0.5) * z * one_plus_u).astype(F32), dtype), u, r


def alu(x, beta=0.5, dtype="bf16"):
    return alu_parts(x, beta, dtype)[0]


def alu_vjp(u, r, g, dtype="bf16"):
    d = (F32(0.5) * (F32(1) + u) + F32(0.5) * u * (r * r)).astype(F32)
    return round_to((np.asarray(g, F32) * d).astype(F32), dtype)


def _mm(a, b, dtype):
    return round_to(np.asarray(a, F32) @ np.asarray(b, F32), dtype)


def ffn_forward(h2, w_g, w_u, w_d, beta=0.5, dtype="bf16"):
    """(out, gate, up, y) of (gate * alu(up)) @ w_d (model.py:185-193)."""
    gate = _mm(h2, round_to(w_g, dtype), dtype)
    up = _mm(h2, round_to(w_u, dtype), dtype)
    act = alu(up, beta, dtype)
    y = round_to(gate * act, dtype)
    return _mm(y, round_to(w_d, dtype), dtype), gate, up, y


def ffn_backward(h2, w_g, w_u, w_d, dout, beta=0.5, dtype="bf16"):
    """(dh2, dw_g, dw_u, dw_d, d_gate, d_up) for the cotangent ``dout`` of the block output."""
    _, gate, up, y = ffn_forward(h2, w_g, w_u, w_d, beta, dtype)
    act, u, r = alu_parts(up, beta, dtype)
    dy = _mm(dout, round_to(w_d, dtype).T, dtype)
    d_gate = round_to(dy * act, dtype)
    d_act = round_to(dy * gate, dtype)
    d_up = alu_vjp(u, r, d_act, dtype)
    dh2 = round_to(np.asarray(d_gate, F32) @ round_to(w_g, dtype).T.astype(F32)
                   + np.asarray(d_up, F32) @ round_to(w_u, dtype).T.astype(F32), dtype)
    dw_g = _mm(np.asarray(h2, F32).T, d_gate, dtype)
    dw_u = _mm(np.asarray(h2, F32).T, d_up, dtype)
    dw_d = _mm(np.asarray(y, F32).T, dout, dtype)
    return dh2, dw_g, dw_u, dw_d, d_gate, d_up
