"""Pins of the attention-prologue oracle (oracle/prologue.py) on the CPU.

* Cayley tables == cos / sin(m * 2 atan w) and exact rotations (tests/test_components.py:59-68).
* float32 RMS norm == float64 closed form; rotation == complex multiplication, norms kept.
* RMS-norm VJP, rotation VJP and the whole chain (norm + gain, rotation, dense algebraic
  attention with a sink) == torch float64 autograd of the closed forms.
* Planted mistakes (gain dropped from the VJP, rotation sign flipped) fail those pins.
"""

import math

import numpy as np
import pytest

from helpers import rel_l2
from oracle import attention as OA
from oracle import prologue as OP

torch = pytest.importorskip("torch")


def test_cayley_tables_are_exact_rotations():
    for head_dim, T in [(64, 300), (128, 2048)]:
        c, s = OP.cayley_table_geometric(head_dim, T)
        half = head_dim // 2
        angles = 2 * np.arctan(0.5 * 1e4 ** (-np.arange(half) / half))
        m = np.arange(T)[:, None]
        # The reference's own bound is 2e-5 at T = 300; the f32 error of the binary powers
        # grows with log2(T) renormalised squarings and the size of m * angle.
        tol = 2e-5 if T <= 300 else 2e-4
        np.testing.assert_allclose(c, np.cos(m * angles), atol=tol)
        np.testing.assert_allclose(s, np.sin(m * angles), atol=tol)
        np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-6)
    c, s = OP.cayley_table_geometric(64, 16, fraction=0.5)
    assert np.all(c[:, 16:] == 1) and np.all(s[:, 16:] == 0)


def test_rms_norm_and_rotary_match_closed_forms():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2, 3, 40, 64)) * 2.5).astype(np.float32)
    g = (1 + 0.3 * rng.standard_normal(64)).astype(np.float32)
    y, tau = OP.rms_norm(x, g, 1e-5, "f32")
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64, -1, keepdims=True) + 1e-5) * g
    assert rel_l2(y, ref) < 1e-6
    c, s = OP.cayley_table_geometric(64, 40)
    r = OP.rotary(y, c, s, "f32")
    z = (y[..., :32] + 1j * y[..., 32:]) * (c + 1j * s)
    assert rel_l2(r, np.concatenate([z.real, z.imag], -1)) < 1e-6
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(y, axis=-1), rtol=1e-5)


def _torch_chain(q, k, v, do, sink, gq, gk, cos, sin, n=16, c=8.0, eps=1e-5):
    """float64 autograd of norm + gain, rotation and the dense algebraic attention."""
    t = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    tq, tk, tv, tgq, tgk, ts = t(q), t(k), t(v), t(gq), t(gk), t(sink)
    cs, sn = torch.tensor(cos, dtype=torch.float64), torch.tensor(sin, dtype=torch.float64)

    def norm(x, g):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * g

    def rot(x):
        h = x.shape[-1] // 2
        x1, x2 = x[..., :h], x[..., h:]
        return torch.cat([x1 * cs - x2 * sn, x1 * sn + x2 * cs], -1)

    qr, kr = rot(norm(tq, tgq)), rot(norm(tk, tgk))
    D = q.shape[-1]
    x = qr @ kr.transpose(-1, -2) / math.sqrt(D) / c
    T = q.shape[-2]
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    logit = torch.where(mask, n * torch.asinh(x), torch.tensor(-math.inf, dtype=torch.float64))
    sink_logit = (n * torch.asinh(ts.reshape(1, -1, 1, 1) / c)).expand(*logit.shape[:-1], 1)
    p = torch.softmax(torch.cat([logit, sink_logit], -1), -1)[..., :-1]
    o = p @ tv
    (o * torch.tensor(do, dtype=torch.float64)).sum().backward()
    g = lambda a: a.grad.numpy()
    return o.detach().numpy(), g(tq), g(tk), g(tv), g(tgq), g(tgk), g(ts)


def _oracle_chain(q, k, v, do, sink, gq, gk, cos, sin, dtype, rms_vjp=OP.rms_norm_vjp):
    q_s, k_r, q_r, tau_q, tau_k = OP.prologue_forward(q, k, gq, gk, cos, sin, dtype=dtype)
    res = OA.flash_attention_oracle(q_r, k_r, v, sink, do, n=16, c=8.0, dtype=dtype)
    assert res["in_range"]
    np.testing.assert_array_equal(res["q_s"], q_s)
    dqn = OP.rotary_vjp(res["dq"], cos, sin, dtype)
    dkn = OP.rotary_vjp(res["dk"], cos, sin, dtype)
    dq, dgq = rms_vjp(q, gq, tau_q, dqn, dtype)
    dk, dgk = rms_vjp(k, gk, tau_k, dkn, dtype)
    return res["o"], dq, dk, res["dv"], dgq, dgk, res["dsink"]


def _inputs(seed=4, B=1, H=2, T=48, D=64):
    rng = np.random.default_rng(seed)
    q, k, v, do = (rng.standard_normal((B, H, T, D)).astype(np.float32) for _ in range(4))
    q, k = q * 3.0, k * 0.7  # raw projections: the norm has work to do
    gq = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    sink = (rng.standard_normal((1, H, 1, 1)) * 0.1).astype(np.float32)
    cos, sin = OP.cayley_table_geometric(D, T)
    return q, k, v, do, sink, gq, gk, cos, sin


def test_prologue_chain_matches_torch_autograd():
    args = _inputs()
    ref = _torch_chain(*args)
    got = _oracle_chain(*args, dtype="f32")
    names = ["o", "dq", "dk", "dv", "dq_gain", "dk_gain", "dsink"]
    errs = {n: rel_l2(np.reshape(a, -1), np.reshape(b, -1)) for n, a, b in zip(names, got, ref)}
    assert max(errs.values()) < 1e-5, errs


def test_prologue_chain_bf16_within_tolerance():
    q, k, v, do, sink, gq, gk, cos, sin = _inputs(seed=6)
    from oracle.numerics import round_bf16
    q, k, v, do = (round_bf16(a) for a in (q, k, v, do))
    ref = _torch_chain(q, k, v, do, sink, gq, gk, cos, sin)
    got = _oracle_chain(q, k, v, do, sink, gq, gk, cos, sin, dtype="bf16")
    names = ["o", "dq", "dk", "dv", "dq_gain", "dk_gain", "dsink"]
    errs = {n: rel_l2(np.reshape(a, -1), np.reshape(b, -1)) for n, a, b in zip(names, got, ref)}
    assert max(errs.values()) < 2e-2, errs


def test_planted_mistakes_fail_the_pins():
    args = _inputs(seed=8)
    ref = _torch_chain(*args)

    def no_gain_vjp(x, gain, tau, dy, dtype):  # drops the gain from the input gradient
        return OP.rms_norm_vjp(x, None, tau, dy, dtype)
    got = _oracle_chain(*args, dtype="f32", rms_vjp=no_gain_vjp)
    assert rel_l2(got[1], ref[1]) > 1e-3

    q, k, v, do, sink, gq, gk, cos, sin = args
    flipped = OP.rotary(np.ones((1, 1, 8, 64), np.float32), cos[:8], -sin[:8], "f32")
    right = OP.rotary(np.ones((1, 1, 8, 64), np.float32), cos[:8], sin[:8], "f32")
    assert rel_l2(flipped, right) > 1e-2
    # A transposed rotation (the transpose used in the forward) breaks the VJP pin.
    dy = np.random.default_rng(1).standard_normal((1, 1, 8, 64)).astype(np.float32)
    tr = torch.tensor(np.ones((1, 1, 8, 64)), dtype=torch.float64, requires_grad=True)
    cs, sn = torch.tensor(cos[:8], dtype=torch.float64), torch.tensor(sin[:8], dtype=torch.float64)
    out = torch.cat([tr[..., :32] * cs - tr[..., 32:] * sn, tr[..., :32] * sn + tr[..., 32:] * cs], -1)
    (out * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    assert rel_l2(OP.rotary_vjp(dy, cos[:8], sin[:8], "f32"), tr.grad.numpy()) < 1e-6
    assert rel_l2(OP.rotary(dy, cos[:8], sin[:8], "f32"), tr.grad.numpy()) > 1e-2
