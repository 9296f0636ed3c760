"""Generate the golden fixtures of the hot path (test infrastructure).

The reference ships no golden vectors (its tests draw inputs from jax.random on the fly), so
the fixtures come from the float64 closed forms the reference's own CPU tests use as ground
truth (tests/test_components.py:27-56): softmax attention over the compressed logits
n*asinh(s/c) with a sink column, and the true NLL of the algebraic head, both differentiated
with torch float64 autograd (oracle/closed_form.py). Inputs are rounded to bf16 first, so
every backend sees exactly the same values. The final RMS norm (algebraic.py:76-83) and the
ALU-GLU block (model.py:185-193, alu at algebraic.py:84-103) get the same treatment: their
defining formulas in torch float64 and autograd, written here and not taken from the oracle.

Usage: python tests/golden/make_golden.py   (rewrites tests/golden/*.npz)
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))            # tests/ (helpers)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root (oracle)

from helpers import attention_inputs, head_inputs  # noqa: E402
from oracle.closed_form import attention_closed_form, head_closed_form  # noqa: E402

# name: (B, H, T, D, sink, seed)
ATTENTION = {
    "attn_b1h2t48d64_sink": (1, 2, 48, 64, True, 21),
    "attn_b1h1t40d128": (1, 1, 40, 128, False, 22),
}
# name: (N, d, V, seed, e_std)
HEAD = {
    "head_n32d64v300": (32, 64, 300, 23, 0.15),
    "head_n24d128v260": (24, 128, 260, 24, 0.05),
}
# name: (rows, d, gain, seed)
NORM = {
    "norm_r16d64_gain": (16, 64, True, 25),
    "norm_r9d40": (9, 40, False, 26),
}
# name: (N, d, F, beta, seed)
FFN = {  # d_ff a multiple of 128, as the fused kernels require
    "ffn_n24d32f128_b05": (24, 32, 128, 0.5, 27),
    "ffn_n20d24f128_b1": (20, 24, 128, 1.0, 28),
}
ATTN_N, ATTN_C = 16, 8.0
HEAD_N, HEAD_C = 8, 2.0
NORM_EPS = 1e-5


def f32(a):
    return np.asarray(a, np.float32)


def make_attention(name, B, H, T, D, sink, seed):
    q, k, v, do, s = attention_inputs(B, H, T, D, seed=seed, sink=sink)
    o, dq, dk, dv, ds = attention_closed_form(q, k, v, s, do, n=ATTN_N, c=ATTN_C)
    arrays = dict(q=q, k=k, v=v, do=do, o=f32(o), dq=f32(dq), dk=f32(dk), dv=f32(dv),
                  n=np.int32(ATTN_N), c=np.float32(ATTN_C))
    if sink:
        arrays.update(sink=f32(s), dsink=f32(ds))
    np.savez(os.path.join(HERE, name + ".npz"), **arrays)


def make_head(name, N, d, V, seed, e_std):
    h, E, t = head_inputs(N, d, V, seed=seed, e_std=e_std)
    nll, pt, dh, dE = head_closed_form(h, E, t, 1.0, n=HEAD_N, c=HEAD_C)
    np.savez(os.path.join(HERE, name + ".npz"), h=h, E=E, targets=t, g=np.float32(1.0),
             nll=np.float64(nll), pt=f32(pt), obj=np.float64(np.mean(1.0 - pt)), dh=f32(dh), dE=f32(dE),
             n=np.int32(HEAD_N), c=np.float32(HEAD_C))


def _bf16(rng, shape, scale=1.0):
    from oracle.numerics import round_bf16
    return round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def make_norm(name, rows, d, gain, seed):
    """y = x rsqrt(mean(x^2) + eps) g, and its VJP for the cotangent dy, in float64."""
    import torch
    rng = np.random.default_rng(seed)
    x, dy = _bf16(rng, (rows, d), 2.0), _bf16(rng, (rows, d))
    g = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32) if gain else None
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tg = torch.tensor(g, dtype=torch.float64, requires_grad=True) if gain else None
    y = tx * torch.rsqrt((tx * tx).mean(-1, keepdim=True) + NORM_EPS)
    if gain:
        y = y * tg
    (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    arrays = dict(x=x, dy=dy, y=f32(y.detach().numpy()), dx=f32(tx.grad.numpy()), eps=np.float32(NORM_EPS))
    if gain:
        arrays.update(gain=g, dgain=f32(tg.grad.numpy()))
    np.savez(os.path.join(HERE, name + ".npz"), **arrays)


def make_ffn(name, N, d, F, beta, seed):
    """out = (h2 w_g * alu(h2 w_u)) w_d with alu(z) = z/2 (1 + b z / sqrt(1 + b^2 z^2)), and the
    gradients of sum(out * dout) in h2 and the three weights, in float64."""
    import torch
    rng = np.random.default_rng(seed)
    h2, dout = _bf16(rng, (N, d)), _bf16(rng, (N, d))
    w_g, w_u = _bf16(rng, (d, F), d ** -0.5), _bf16(rng, (d, F), d ** -0.5)
    w_d = _bf16(rng, (F, d), F ** -0.5)
    t = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (h2, w_g, w_u, w_d)]
    up = t[0] @ t[2]
    act = 0.5 * up * (1 + beta * up / torch.sqrt(1 + (beta * up) ** 2))
    out = ((t[0] @ t[1]) * act) @ t[3]
    (out * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    np.savez(os.path.join(HERE, name + ".npz"), h2=h2, w_g=w_g, w_u=w_u, w_d=w_d, dout=dout,
             beta=np.float32(beta), out=f32(out.detach().numpy()), dh2=f32(t[0].grad.numpy()),
             dw_g=f32(t[1].grad.numpy()), dw_u=f32(t[2].grad.numpy()), dw_d=f32(t[3].grad.numpy()))


def main():
    for name, cfg in ATTENTION.items():
        make_attention(name, *cfg)
    for name, cfg in HEAD.items():
        make_head(name, *cfg)
    for name, cfg in NORM.items():
        make_norm(name, *cfg)
    for name, cfg in FFN.items():
        make_ffn(name, *cfg)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
