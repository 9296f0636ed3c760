"""GPU parity of the fused head on float32 hidden states (csrc/head_f32.hip).

fused_head.py:168 casts E to h's dtype and the model's compute dtype is a parameter
(model.py:57), so a float32 model reaches the head with f32 h. The reference then runs its
whole head in f32 (no bf16 rounding), so the HIP f32 path is held to f32 bars against the
float64 dense oracle (``oracle.head.dense_forward`` / ``dense_backward``, pinned to the true
NLL gradient in tests/test_oracle.py): objective and telemetry within 1e-5 relative, dh and
dE within 1e-5 relative L2, and the eval head's log p within 1e-5 absolute of
``oracle.head.eval_logprob``. Inputs are f32 values that are not bf16-representable, so a
hidden bf16 cast anywhere on the path would fail the bars.
"""

import numpy as np
import pytest

from helpers import rel_l2
from oracle import head as OH

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _inputs(N, d, V, seed, e_std=0.15, h_scale=1.0):
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((N, d)) * h_scale).astype(np.float32)
    E = (rng.standard_normal((V, d)) * e_std).astype(np.float32)
    t = rng.integers(0, V, N).astype(np.int32)
    return h, E, t


def _run(h, E, t, n, c, e_dtype=torch.float32, g=1.0):
    from algebraic_amd.kernels.fused_head import fused_head
    th = torch.tensor(h, device="cuda", requires_grad=True)
    tE = torch.tensor(E, device="cuda").to(e_dtype).requires_grad_(True)
    obj, pt = fused_head(th, tE, torch.tensor(t, device="cuda"), kind="alg_ce", n=n, c=c)
    (obj * g).backward()
    torch.cuda.synchronize()
    assert th.grad.dtype == torch.float32 and tE.grad.dtype == e_dtype
    f = lambda x: x.detach().float().cpu().numpy().astype(np.float64)
    return float(obj.detach()), f(pt), f(th.grad), f(tE.grad)


SHAPES = [  # (N, d, V)
    (256, 128, 300),
    (128, 128, 517),     # ragged vocabulary
    (100, 128, 260),     # N below one token tile
    (384, 256, 1000),    # N not a multiple of 128
    (256, 72, 333),      # d not a multiple of the k step
    (1024, 256, 4096),   # the reference's head-test shape (vocabulary split of dh)
]


@pytest.mark.parametrize("schedule", ["recompute", "streamed"])
@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_head_f32_matches_dense(shape, n, c, schedule, monkeypatch):
    """"streamed" runs 256-row vocabulary chunks, dh accumulated over them in f32."""
    from algebraic_amd.kernels import fused_head as FH
    monkeypatch.setattr(FH, "SCHEDULE", schedule)
    monkeypatch.setattr(FH, "VOCAB_CHUNK", 256)
    N, d, V = shape
    h, E, t = _inputs(N, d, V, seed=N + d + V + n)
    print(f"f32 head N{N} d{d} V{V} n{n} {schedule}", flush=True)
    obj, pt, dh, dE = _run(h, E, t, n, c, g=0.7)
    obj_r, pt_r = OH.dense_forward(h, E, t, n=n, c=c)
    dh_r, dE_r = OH.dense_backward(h, E, t, 0.7, n=n, c=c)
    np.testing.assert_allclose(obj, obj_r, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(pt, pt_r, rtol=1e-5, atol=1e-9)
    assert rel_l2(dh, dh_r) < 1e-5
    assert rel_l2(dE, dE_r) < 1e-5


def test_head_f32_model_widths():
    """The reference's production widths (test_fused_head_tpu.py:51-70: 256 tokens, V 32768,
    E ~ 0.02 N(0, 1)) at d = 1024."""
    h, E, t = _inputs(256, 1024, 32768, seed=1066, e_std=0.02)
    obj, pt, dh, dE = _run(h, E, t, 8, 2.0)
    obj_r, pt_r = OH.dense_forward(h, E, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, E, t, 1.0, n=8, c=2.0)
    np.testing.assert_allclose(obj, obj_r, rtol=1e-5)
    np.testing.assert_allclose(pt, pt_r, rtol=1e-5, atol=1e-12)
    assert rel_l2(dh, dh_r) < 1e-5
    assert rel_l2(dE, dE_r) < 1e-5


def test_head_f32_with_bf16_embedding():
    """f32 h with a bf16 embedding: E is cast to f32 (exactly), and dE comes back in the
    embedding's dtype, bf16 (fused_head.py:254): dh at the f32 bar, dE at bf16 rounding."""
    h, E, t = _inputs(256, 128, 1000, seed=5)
    Eb = torch.tensor(E).to(torch.bfloat16).float().numpy()
    obj, pt, dh, dE = _run(h, Eb, t, 8, 2.0, e_dtype=torch.bfloat16)
    obj_r, _ = OH.dense_forward(h, Eb, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, Eb, t, 1.0, n=8, c=2.0)
    np.testing.assert_allclose(obj, obj_r, rtol=1e-5)
    assert rel_l2(dh, dh_r) < 1e-5
    assert rel_l2(dE, dE_r) < 4e-3  # one bf16 rounding of the f32 gradient


def test_head_f32_confident_targets():
    """Confident predictions (median p_t about 0.99, target rows aligned with the hidden
    states). The target entry of dZ = s (p - y) r cancels in f32, in the reference's f32
    computation as here, to a relative error of about eps / (1 - p_t) (1e-5 at this p_t), so
    the bars are 1e-4."""
    h, E, t = _inputs(256, 128, 512, seed=12, e_std=0.02)
    E[t] = h * 0.03
    obj, pt, dh, dE = _run(h, E, t, 8, 2.0)
    obj_r, pt_r = OH.dense_forward(h, E, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, E, t, 1.0, n=8, c=2.0)
    assert 0.98 < np.median(pt_r) < 0.999
    np.testing.assert_allclose(obj, obj_r, rtol=1e-4)
    np.testing.assert_allclose(pt, pt_r, rtol=1e-5)
    assert rel_l2(dh, dh_r) < 1e-4
    assert rel_l2(dE, dE_r) < 1e-4


@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_logprob_f32(n, c):
    from algebraic_amd.kernels.fused_head import head_logprob
    N, d, V = 384, 256, 5000
    h, E, t = _inputs(N, d, V, seed=77 + n)
    lp, am = head_logprob(torch.tensor(h, device="cuda"), torch.tensor(E, device="cuda"),
                          torch.tensor(t, device="cuda"), n=n, c=c)
    lp_r, am_r, z = OH.eval_logprob(h, E, t, n=n, c=c)
    np.testing.assert_allclose(lp.cpu().numpy(), lp_r, atol=1e-5, rtol=0)
    am = am.cpu().numpy()
    zr = z[np.arange(N), am]
    np.testing.assert_allclose(zr, z.max(axis=1), rtol=1e-6, atol=1e-6)  # the largest logit up to f32 ties
    assert (am == am_r).mean() > 0.99
