"""GPU parity of the ALU-GLU feed-forward with fused activation epilogues (`alu_glu_ffn`,
C ABI alg_ffn_alu_glu_fwd / _dy) against the oracle (oracle/ffn.py, pinned by
tests/test_ffn_oracle.py): model.py:185-193, algebraic.py:86-113.

Bars (relative L2): output and every gradient within 1e-2 of the cast-faithful oracle, the
fused epilogue outputs (y, gate, up, [d_gate | d_up]) within 5e-3; at the 1b shape
(N 16384, d 1536, d_ff 4224) sampled token rows of y/gate/up and [d_gate | d_up] against the
oracle restricted to those rows.
"""

import numpy as np
import pytest

from helpers import rel_l2
from oracle import ffn as OF
from oracle.numerics import round_bf16

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _inputs(N, d, F, dm, seed):
    rng = np.random.default_rng(seed)
    r = lambda *s, sc=1.0: round_bf16((rng.standard_normal(s) * sc).astype(np.float32))
    return r(N, d), r(d, F, sc=d ** -0.5), r(d, F, sc=d ** -0.5), r(F, dm, sc=F ** -0.5), r(N, dm)


def _dev(a):
    return torch.tensor(a, device="cuda").to(torch.bfloat16)


@pytest.mark.parametrize("N,d,F,beta", [(256, 128, 256, 0.5), (300, 256, 384, 0.5), (512, 384, 1024, 0.5),
                                         (200, 72, 128, 0.5), (300, 256, 384, 1.0), (200, 72, 128, 0.8)])
def test_ffn_matches_oracle(N, d, F, beta):
    """beta 0.5 is the model's SiLU-matched slope, 1.0 the reference's default (algebraic.py:97)
    and 0.8 its GELU-matched one."""
    from algebraic_amd.kernels.ffn import alu_glu_ffn
    h2, w_g, w_u, w_d, dout = _inputs(N, d, F, d, seed=N + F)
    print(f"[ffn] N={N} d={d} F={F} beta={beta}", flush=True)
    t = [_dev(a).requires_grad_(True) for a in (h2, w_g, w_u, w_d)]
    out = alu_glu_ffn(*t, beta=beta)
    out.backward(_dev(dout))
    torch.cuda.synchronize()
    o_ref, _, _, _ = OF.ffn_forward(h2, w_g, w_u, w_d, beta)
    dh2, dw_g, dw_u, dw_d, _, _ = OF.ffn_backward(h2, w_g, w_u, w_d, dout, beta)
    g = lambda x: x.detach().float().cpu().numpy()
    errs = {"out": rel_l2(g(out), o_ref), "dh2": rel_l2(g(t[0].grad), dh2), "dw_g": rel_l2(g(t[1].grad), dw_g),
            "dw_u": rel_l2(g(t[2].grad), dw_u), "dw_d": rel_l2(g(t[3].grad), dw_d)}
    print(f"  {errs}", flush=True)
    assert max(errs.values()) < 1e-2, errs


def _abi_fwd(h2, w_gu, N, d, F, beta=0.5):
    from algebraic_amd import _lib as L
    lib = L.load()
    y, gate, up = (torch.empty((N, F), dtype=torch.bfloat16, device="cuda") for _ in range(3))
    L.check(lib.alg_ffn_alu_glu_fwd(L.stream_of(h2), N, d, F, L.ptr(h2), L.ptr(w_gu), beta, L.ptr(y), L.ptr(gate),
                                    L.ptr(up)), "ffn fwd")
    return y, gate, up


def _abi_dy(dout, w_d, gate, up, N, dm, F, beta=0.5):
    from algebraic_amd import _lib as L
    lib = L.load()
    d_gu = torch.empty((N, 2 * F), dtype=torch.bfloat16, device="cuda")
    L.check(lib.alg_ffn_alu_glu_dy(L.stream_of(dout), N, dm, F, L.ptr(dout), L.ptr(w_d), L.ptr(gate), L.ptr(up),
                                   beta, L.ptr(d_gu)), "ffn dy")
    return d_gu


@pytest.mark.parametrize("N,d,F", [(300, 256, 384), (16384, 1536, 4224)])
def test_ffn_fused_epilogues_sampled_rows(N, d, F):
    """The fused products' outputs on sampled token rows (incl. the last, ragged tile) against
    the oracle on those rows; at the second shape this is the 1b model's FFN (d_ff 4224)."""
    h2, w_g, w_u, w_d, dout = _inputs(N, d, F, d, seed=7)
    print(f"[ffn] fused epilogues N={N} d={d} F={F}", flush=True)
    th2, tdo, twd = _dev(h2), _dev(dout), _dev(w_d)
    w_gu = _dev(np.concatenate([w_g, w_u], axis=1))
    y, gate, up = _abi_fwd(th2, w_gu, N, d, F)
    d_gu = _abi_dy(tdo, twd, gate, up, N, d, F)
    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, 30)]))
    _, g_ref, u_ref, y_ref = OF.ffn_forward(h2[rows], w_g, w_u, w_d, 0.5)
    act, u, r = OF.alu_parts(u_ref, 0.5)
    dy = round_bf16(dout[rows] @ w_d.T)
    dg_ref = round_bf16(dy * act)
    du_ref = OF.alu_vjp(u, r, round_bf16(dy * g_ref))
    g = lambda x: x.float().cpu().numpy()[rows]
    errs = {"gate": rel_l2(g(gate), g_ref), "up": rel_l2(g(up), u_ref), "y": rel_l2(g(y), y_ref),
            "d_gate": rel_l2(g(d_gu)[:, :F], dg_ref), "d_up": rel_l2(g(d_gu)[:, F:], du_ref)}
    print(f"  {errs}", flush=True)
    assert max(errs.values()) < 5e-3, errs
