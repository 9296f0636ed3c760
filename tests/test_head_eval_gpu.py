"""GPU parity of the streamed evaluation head (`head_logprob`, C ABI `alg_head_eval`): the
scorer's per-token log p(target) and argmax (src/algebraic/benchmarking.py:178-188,
src/algebraic/evaluation.py:13-23, head "alg_ce") without the (N, V) logits.

Bars: log-probabilities within 1e-4 absolute (they are about -log V) of the float64 dense
oracle; the argmax index holds the largest float64 logit up to a near-tie (1e-5 relative)
and equals the oracle's argmax on at least 99 % of the tokens; at full size (C2, C4b) the same
against a float64 dense evaluation on the device; and log p == log(pt) of the training
head's telemetry (both from the same stream of logits).
"""

import numpy as np
import pytest

from helpers import head_inputs
from oracle import head as OH

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CASES = [(256, 128, 300), (384, 256, 1000), (100, 128, 260), (512, 512, 2304), (256, 72, 333)]


def _run(h, E, t, n=8, c=2.0):
    from algebraic_amd.kernels.fused_head import head_logprob
    th = torch.tensor(h, device="cuda").to(torch.bfloat16)
    tE = torch.tensor(E, device="cuda").to(torch.bfloat16)
    lp, am = head_logprob(th, tE, torch.tensor(t, device="cuda"), n=n, c=c)
    torch.cuda.synchronize()
    return lp.cpu().numpy().astype(np.float64), am.cpu().numpy()


def _check_argmax(am, z, frac=0.99):
    best = z.max(axis=1)
    got = z[np.arange(len(am)), am]
    assert np.all(got >= best - 1e-5 * (np.abs(best) + 1)), "argmax is not a (near-)maximum"
    agree = float(np.mean(am == np.argmax(z, axis=1)))
    assert agree >= frac, f"argmax agrees on {agree:.4f} of tokens"
    return agree


@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_logprob_matches_oracle(shape, n, c):
    N, d, V = shape
    h, E, t = head_inputs(N, d, V, seed=17, e_std=0.05)
    print(f"[eval head] {shape} n={n} c={c}", flush=True)
    lp, am = _run(h, E, t, n, c)
    lp_ref, am_ref, z = OH.eval_logprob(h, E, t, n=n, c=c)
    err = float(np.max(np.abs(lp - lp_ref)))
    print(f"  max |logprob - oracle| = {err:.2e}", flush=True)
    assert err < 1e-4
    _check_argmax(am, z)


def test_head_logprob_is_log_of_training_telemetry():
    from algebraic_amd.kernels.fused_head import fused_head
    h, E, t = head_inputs(512, 256, 4096, seed=19)
    lp, _ = _run(h, E, t)
    _, tel = fused_head(torch.tensor(h, device="cuda").to(torch.bfloat16),
                        torch.tensor(E, device="cuda").to(torch.bfloat16), torch.tensor(t, device="cuda"),
                        kind="alg_ce", n=8, c=2.0)
    np.testing.assert_allclose(lp, np.log(tel.cpu().numpy().astype(np.float64)), atol=2e-5)


@pytest.mark.parametrize("shape", [(8192, 768, 50257), (16384, 2048, 32000)])
def test_head_logprob_full_size(shape):
    """C2 and C4b: every token against log_softmax(n asinh(z/c)) and argmax of float64
    logits formed on the device (torch float64 products of the same bf16 inputs)."""
    N, d, V = shape
    h, E, t = head_inputs(N, d, V, seed=2)
    print(f"[eval head] full size {shape}", flush=True)
    lp, am = _run(h, E, t)
    h64 = torch.tensor(h, device="cuda", dtype=torch.float64)
    E64 = torch.tensor(E, device="cuda", dtype=torch.float64)
    tt = torch.tensor(t, device="cuda", dtype=torch.long)
    lps, ams, gaps = [], [], []
    for s in range(0, N, 2048):
        z = h64[s:s + 2048] @ E64.t()
        a = 8 * torch.asinh(z / 2.0)
        lps.append((a.gather(1, tt[s:s + 2048, None])[:, 0] - torch.logsumexp(a, 1)).cpu())
        ams.append(torch.argmax(z, 1).cpu())
        sel = z.gather(1, torch.tensor(am[s:s + 2048], device="cuda")[:, None])[:, 0]
        gaps.append((z.max(1).values - sel).cpu() / (z.max(1).values.abs().cpu() + 1))
        del z, a
    lp_ref = torch.cat(lps).numpy()
    err = float(np.max(np.abs(lp - lp_ref)))
    agree = float(np.mean(am == torch.cat(ams).numpy()))
    gap = float(torch.cat(gaps).max())
    print(f"  max |logprob - float64| = {err:.2e}, argmax agreement {agree:.5f}, worst gap {gap:.1e}", flush=True)
    assert err < 1e-4 and agree >= 0.99 and gap <= 1e-5


def test_out_of_range_targets_read_a_zero_logit():
    """A target outside [0, V) contributes no column (fused_head.py:87 sums none), so its
    logit reads 0: the training head's telemetry is rho(0)^n stat^n = 1/l and the eval head's
    log p is -log l, with l (and stat) unchanged from a run with valid targets. Covers the
    interior and the edge vocabulary tiles (V not a multiple of the tile)."""
    from algebraic_amd.kernels.fused_head import fused_head, head_logprob
    N, d, V = 512, 256, 1000
    h, E, t = head_inputs(N, d, V, seed=23)
    bad = t.copy()
    bad[::7] = -1
    bad[3::7] = V
    bad[5::7] = V + 37
    invalid = (bad < 0) | (bad >= V)
    stat, _, pt_ref, _ = OH.kernel_forward(h, E, t, n=8, c=2.0)
    th = torch.tensor(h, device="cuda").to(torch.bfloat16)
    tE = torch.tensor(E, device="cuda").to(torch.bfloat16)
    tb = torch.tensor(bad, device="cuda")
    _, tel = fused_head(th, tE, tb, kind="alg_ce", n=8, c=2.0)
    lp, _ = head_logprob(th, tE, tb, n=8, c=2.0)
    torch.cuda.synchronize()
    tel = tel.cpu().numpy().astype(np.float64)
    lp = lp.cpu().numpy().astype(np.float64)
    st = stat.astype(np.float64)
    np.testing.assert_allclose(tel[invalid], st[invalid] ** 8, rtol=2e-5)
    np.testing.assert_allclose(lp[invalid], 8 * np.log(st[invalid]), atol=2e-5)
    np.testing.assert_allclose(tel[~invalid], pt_ref[~invalid], rtol=1e-4, atol=1e-9)


@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_logprob_logits_beyond_the_training_clamp(n, c):
    """The scorer's log_softmax(n asinh(z/c)) has no clamp (src/algebraic/evaluation.py:13-23).
    One embedding row is aligned with token 0's hidden state so that logit reaches several times
    c X (X = 1/4 (1e38/V)^(1/n), the training head's clamp), and through it the other tokens see
    large positive and negative logits: log p and the argmax against the float64 oracle."""
    from oracle.numerics import head_clamp, round_bf16
    N, d, V = 256, 256, 1000
    h, E, t = head_inputs(N, d, V, seed=29, e_std=0.05)
    big = 4.0 * c * head_clamp(V, n)
    E[7] = round_bf16(h[0] * np.float32(big / d))
    t[0] = 7
    lp, am = _run(h, E, t, n, c)
    lp_ref, _, z = OH.eval_logprob(h, E, t, n=n, c=c)
    assert z[0, 7] > 3.0 * c * head_clamp(V, n) and z[:, 7].min() < -c * head_clamp(V, n) / 10
    err = float(np.max(np.abs(lp - lp_ref)))
    print(f"  logit max {z.max():.0f} (c X = {c * head_clamp(V, n):.0f}): max |logprob - oracle| = {err:.2e}",
          flush=True)
    assert err < 1e-4
    _check_argmax(am, z)


def test_head_argmax_takes_the_first_nan():
    """jnp.argmax returns the first NaN's index: a token whose hidden state is NaN has only NaN
    logits (argmax 0, log p NaN); an embedding row of NaN gives every token a NaN logit there."""
    N, d, V = 256, 128, 700
    h, E, t = head_inputs(N, d, V, seed=31)
    h[5] = np.nan
    lp, am = _run(h, E, t)
    assert am[5] == 0 and np.isnan(lp[5])
    assert np.isfinite(lp[np.arange(N) != 5]).all()
    E[300] = np.nan
    lp, am = _run(h, E, t)
    assert am[5] == 0
    np.testing.assert_array_equal(am[np.arange(N) != 5], 300)
