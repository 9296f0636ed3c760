"""Generate the golden fixtures of the attention and head hot path (test infrastructure).

The reference ships no golden vectors (its tests draw inputs from jax.random on the fly), so
the fixtures come from the float64 closed forms the reference's own CPU tests use as ground
truth (tests/test_components.py:27-56): softmax attention over the compressed logits
n*asinh(s/c) with a sink column, and the true NLL of the algebraic head, both differentiated
with torch float64 autograd (oracle/closed_form.py). Inputs are rounded to bf16 first, so
every backend sees exactly the same values.

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
ATTN_N, ATTN_C = 16, 8.0
HEAD_N, HEAD_C = 8, 2.0


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


def main():
    for name, cfg in ATTENTION.items():
        make_attention(name, *cfg)
    for name, cfg in HEAD.items():
        make_head(name, *cfg)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
