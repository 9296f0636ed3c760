"""GPU parity on the reference's own fused-head test cases (tests/test_fused_head_tpu.py).

The reference compares its Pallas head with a dense JAX head on the same inputs; here the HIP
head (through the ``fused_head`` mirror) is compared with this build's float64 dense oracle of
the lean likelihood (``oracle.head.dense_forward`` / ``dense_backward``, pinned to the true
NLL gradient), with the reference's shapes, input distributions and tolerances. Inputs come
from numpy's seeded generator; E is passed in float32 as there, cast to the hidden dtype
inside the head (fused_head.py:168), and dE comes back in float32.

  test_fused_head_matches_dense            :14-48  (alg_ce, (n, c) in {(16, 16), (8, 2)},
                                                    V in {32768, 4096}, N 1024, d 256,
                                                    E ~ 0.15 N(0, 1))
  test_production_head_tiles_at_model_widths :51-70 (alg_ce, d in {1024, 1536}, 256 tokens,
                                                    V 32768, E ~ 0.02 N(0, 1))
``kind="ce"`` is the softmax control arm, outside the built path.
"""

import numpy as np
import pytest

from oracle import head as OH
from oracle.numerics import round_bf16

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _run(h, E, t, n, c, **kw):
    from algebraic_amd.kernels.fused_head import fused_head
    th = torch.tensor(h, device="cuda").to(torch.bfloat16).requires_grad_(True)
    tE = torch.tensor(E, device="cuda", dtype=torch.float32, requires_grad=True)
    obj, tel = fused_head(th, tE, torch.tensor(t, device="cuda"), kind="alg_ce", n=n, c=c, **kw)
    dh, dE = torch.autograd.grad(obj, (th, tE))
    assert dE.dtype == torch.float32
    return (float(obj.detach()), tel.cpu().numpy().astype(np.float64), dh.float().cpu().numpy().astype(np.float64),
            dE.cpu().numpy().astype(np.float64))


def _inputs(seed, N, d, V, e_std):
    rng = np.random.default_rng(seed)
    h = round_bf16(rng.standard_normal((N, d)).astype(np.float32))
    E = (rng.standard_normal((V, d)) * e_std).astype(np.float32)
    t = rng.integers(0, V, N).astype(np.int32)
    return h, E, t


@pytest.mark.parametrize("n,c", [(16, 16.0), (8, 2.0)])
@pytest.mark.parametrize("V", [32768, 4096])
def test_fused_head_matches_dense(n, c, V):
    N, d = 1024, 256
    h, E, t = _inputs(100 + V + n, N, d, V, 0.15)
    obj, tel, dh, dE = _run(h, E, t, n, c, block_n=256, block_v=1024)
    Eb = round_bf16(E)  # the cast to the hidden dtype (fused_head.py:168)
    obj_r, pt_r = OH.dense_forward(h, Eb, t, n=n, c=c)
    dh_r, dE_r = OH.dense_backward(h, Eb, t, 1.0, n=n, c=c)
    np.testing.assert_allclose(obj, obj_r, rtol=2e-3, atol=2e-4)
    np.testing.assert_allclose(tel, pt_r, rtol=2e-2, atol=2e-4)
    for a, b in ((dh, dh_r), (dE, dE_r)):
        scale = np.abs(b).max() + 1e-12
        np.testing.assert_allclose(a / scale, b / scale, atol=2e-2)
        cos = (a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum())
        assert cos > 0.999


@pytest.mark.parametrize("width", [1024, 1536])
def test_production_head_tiles_at_model_widths(width):
    tokens, vocab = 256, 32768
    h, E, t = _inputs(42 + width, tokens, width, vocab, 0.02)
    obj, tel, dh, dE = _run(h, E, t, 8, 2.0)
    Eb = round_bf16(E)
    obj_r, pt_r = OH.dense_forward(h, Eb, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, Eb, t, 1.0, n=8, c=2.0)
    np.testing.assert_allclose(obj, obj_r, rtol=0.002, atol=0.0002)
    np.testing.assert_allclose(tel, pt_r, rtol=0.02, atol=2e-7)
    for a, b in ((dh, dh_r), (dE, dE_r)):
        assert np.linalg.norm(a - b) / np.linalg.norm(b) < 0.01
