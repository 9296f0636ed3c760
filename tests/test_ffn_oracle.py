"""Pins of the ALU-GLU oracle (oracle/ffn.py) on the CPU: the activation and its VJP against
the closed form and torch float64 autograd (tests/test_components.py:71-78), the negative
tail, and the whole block's gradients against torch float64 autograd (float32 mode)."""

import numpy as np
import pytest

from helpers import rel_l2
from oracle import ffn as OF

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("beta", [1.0, 0.5])
def test_alu_and_vjp_match_closed_form(beta):
    x = np.linspace(-40, 40, 2001).astype(np.float32)
    ref = 0.5 * x.astype(np.float64) * (1 + beta * x / np.sqrt(1 + (beta * x.astype(np.float64)) ** 2))
    y, u, r = OF.alu_parts(x, beta, "f32")
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-30)
    tx = torch.tensor(x.astype(np.float64), requires_grad=True)
    (0.5 * tx * (1 + beta * tx / torch.sqrt(1 + (beta * tx) ** 2))).sum().backward()
    g = OF.alu_vjp(u, r, np.ones_like(x), "f32")
    # float32 restatement of the reference's derivative 0.5 (1 + u) + 0.5 u r^2: in the negative
    # tail (u -> -1) the sum cancels, leaving f32-rounding-level absolute error (the reference's
    # own test runs in float64, rtol 1e-9 / atol 1e-12).
    np.testing.assert_allclose(g, tx.grad.numpy(), rtol=2e-6, atol=3e-7)


def test_alu_negative_tail_keeps_precision():
    """For x -> -inf, alu(x) -> -1/(4 b^2 x) > 0; the r^2/(1-u) form keeps it, 1 + u cancels."""
    x = np.array([-1e3, -1e4], np.float32)
    y = OF.alu(x, 0.5, "f32")
    ref = 0.5 * x.astype(np.float64) * (1 + 0.5 * x / np.sqrt(1 + (0.5 * x.astype(np.float64)) ** 2))
    np.testing.assert_allclose(y, ref, rtol=1e-4)
    naive = 0.5 * x * (np.float32(1) + (0.5 * x) / np.sqrt(np.float32(1) + (0.5 * x) ** 2))
    assert np.max(np.abs(naive - ref) / np.abs(ref)) > 1e-2  # the cancellation the reference avoids


def test_ffn_block_gradients_match_torch_autograd():
    rng = np.random.default_rng(5)
    N, d, F = 24, 32, 48
    h2, w_g, w_u, w_d, dout = (rng.standard_normal(s).astype(np.float32) * sc for s, sc in
                               [((N, d), 1.0), ((d, F), 0.2), ((d, F), 0.2), ((F, d), 0.2), ((N, d), 1.0)])
    dh2, dw_g, dw_u, dw_d, _, _ = OF.ffn_backward(h2, w_g, w_u, w_d, dout, 0.5, "f32")
    t = lambda a: torch.tensor(a.astype(np.float64), requires_grad=True)
    th, tg, tu, td = t(h2), t(w_g), t(w_u), t(w_d)
    up = th @ tu
    act = 0.5 * up * (1 + 0.5 * up / torch.sqrt(1 + (0.5 * up) ** 2))
    out = ((th @ tg) * act) @ td
    (out * torch.tensor(dout.astype(np.float64))).sum().backward()
    for name, a, b in [("dh2", dh2, th.grad), ("dw_g", dw_g, tg.grad), ("dw_u", dw_u, tu.grad), ("dw_d", dw_d, td.grad)]:
        assert rel_l2(a, b.numpy()) < 1e-5, name
    out_o, *_ = OF.ffn_forward(h2, w_g, w_u, w_d, 0.5, "f32")
    assert rel_l2(out_o, out.detach().numpy()) < 1e-6


@pytest.mark.parametrize("mistake", ["drop_r2_term", "transposed_gate_up"])
def test_planted_mistakes_fail_the_pins(mistake, monkeypatch):
    """Plausible slips planted in the oracle (the derivative without its 0.5 u r^2 term; gate
    and up weights swapped in the backward) must fail the float64 autograd pin above."""
    rng = np.random.default_rng(7)
    N, d, F = 24, 32, 48
    h2, w_g, w_u, w_d, dout = (rng.standard_normal(s).astype(np.float32) * sc for s, sc in
                               [((N, d), 1.0), ((d, F), 0.4), ((d, F), 0.4), ((F, d), 0.2), ((N, d), 1.0)])
    if mistake == "drop_r2_term":
        monkeypatch.setattr(OF, "alu_vjp", lambda u, r, g, dtype="bf16":
                            OF.round_to((np.asarray(g, np.float32) * np.float32(0.5) * (1 + u)).astype(np.float32), dtype))
        dh2, dw_g, dw_u, dw_d, _, _ = OF.ffn_backward(h2, w_g, w_u, w_d, dout, 0.5, "f32")
    else:
        dh2, dw_g, dw_u, dw_d, _, _ = OF.ffn_backward(h2, w_u, w_g, w_d, dout, 0.5, "f32")
    t = lambda a: torch.tensor(a.astype(np.float64), requires_grad=True)
    th, tg, tu, td = t(h2), t(w_g), t(w_u), t(w_d)
    up = th @ tu
    act = 0.5 * up * (1 + 0.5 * up / torch.sqrt(1 + (0.5 * up) ** 2))
    (((th @ tg) * act) @ td * torch.tensor(dout.astype(np.float64))).sum().backward()
    worst = max(rel_l2(a, b.numpy()) for a, b in [(dh2, th.grad), (dw_u, tu.grad)])
    assert worst > 1e-3, f"planted mistake {mistake} passes the pin ({worst:.1e})"
