"""CPU: pin the oracle against closed forms (tests/test_components.py pattern) and tiny brute force.

Every oracle function is checked against something it does not share code with:
* rho / int_pow / inv_root / bf16 rounding against numpy/torch primitives;
* dense attention forward against softmax of n*asinh(s/c) (test_components.py:27-40) and a
  pure-Python loop; its backward against torch float64 autograd of that closed form;
* the kernel-faithful restatement against the dense oracle, in and out of range;
* the head's gradient against torch autograd of the true NLL (test_components.py:43-56).
A planted mistake (dropped sink term, wrong slope) must fail these checks.
"""

import math

import numpy as np
import pytest

from helpers import attention_inputs, head_inputs, rel_l2
from oracle import attention as OA
from oracle import closed_form as CF
from oracle import head as OH
from oracle.numerics import round_bf16
from oracle import numerics as N

torch = pytest.importorskip("torch")


def test_rho_identities():
    x = np.linspace(-50, 50, 1001)
    y = np.linspace(-3, 7, 1001)
    np.testing.assert_allclose(N.rho(x), np.exp(np.arcsinh(x)), rtol=1e-12)
    np.testing.assert_allclose(N.rho(x) * N.rho(-x), 1.0, rtol=1e-12)
    oplus = x * np.sqrt(1 + y * y) + y * np.sqrt(1 + x * x)
    np.testing.assert_allclose(N.rho(x) * N.rho(y), N.rho(oplus), rtol=1e-10)
    rf, r = N.rho_fast(np.linspace(-2, 30, 101))
    np.testing.assert_allclose(rf, np.exp(np.arcsinh(np.linspace(-2, 30, 101))), rtol=1e-12)


@pytest.mark.parametrize("n", [1, 2, 3, 8, 16, 17, 32])
def test_int_pow_and_inv_root(n):
    x = np.linspace(0.3, 3.0, 50)
    np.testing.assert_allclose(N.int_pow(x, n), x ** n, rtol=1e-13)
    if n & (n - 1) == 0 and n > 1:
        np.testing.assert_allclose(N.inv_root(x, n), x ** (-1.0 / n), rtol=1e-13)


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-20, 20, 100000)).astype(np.float32)
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(N.round_bf16(x), ref)


def test_clamps_match_reference_constants():
    # flash.py:747-748 (T=512/1024/2048/16384) and fused_head.py:273 (V=50257/32000), n = 16 / 8
    assert [round(N.attn_clamp(T, 16), 1) for T in (512, 1024, 2048, 16384)] == [69.5, 66.6, 63.7, 56.0]
    assert round(N.head_clamp(50257, 8)) == 3633 and round(N.head_clamp(32000, 8)) == 3844


@pytest.mark.parametrize("n,c", [(8, 1.0), (16, 16.0), (32, 4.0), (16, 8.0)])
def test_dense_weights_are_softmax_of_compressed_logits(n, c):
    rng = np.random.default_rng(0)
    s = rng.standard_normal((2, 3, 7, 7)) * 5
    mask = np.tril(np.ones((7, 7), bool))
    b = np.full((3,), 0.7)
    # oracle weights via _dense_probs with q = s*sqrt(D), k = identity rows (D = T = 7)
    q = s * math.sqrt(7)
    k = np.broadcast_to(np.eye(7), (2, 3, 7, 7))
    p, psink, _ = OA._dense_probs(q, k, n, c, b)
    logits = np.where(mask, n * np.arcsinh(s / c), -np.inf)
    col = np.broadcast_to(n * np.arcsinh(b / c)[None, :, None, None], (2, 3, 7, 1))
    full = np.concatenate([logits, col], -1)
    full = np.exp(full - full.max(-1, keepdims=True))
    ref = full / full.sum(-1, keepdims=True)
    np.testing.assert_allclose(p, ref[..., :-1], rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(psink, ref[..., -1], rtol=1e-10, atol=1e-14)
    big, _, _ = OA._dense_probs(q * 1e6, k, n, c, None)
    assert np.all(np.isfinite(big)) and np.allclose(big.sum(-1), 1.0)


@pytest.mark.parametrize("n,c", [(16, 8.0), (8, 1.0), (32, 4.0)])
@pytest.mark.parametrize("with_sink", [True, False])
def test_dense_attention_vjp_matches_torch_autograd(n, c, with_sink):
    rng = np.random.default_rng(1)
    B, H, T, D = 2, 3, 17, 8
    q, k, v, do = (rng.standard_normal((B, H, T, D)) * 1.5 for _ in range(4))
    sink = rng.standard_normal((1, H, 1, 1)) * 0.5 if with_sink else None
    o_ref, dq_r, dk_r, dv_r, ds_r = CF.attention_closed_form(q, k, v, sink, do, n=n, c=c)
    np.testing.assert_allclose(OA.dense_forward(q, k, v, sink, n=n, c=c), o_ref, rtol=1e-10, atol=1e-12)
    dq, dk, dv, ds = OA.dense_backward(q, k, v, sink, do, n=n, c=c)
    for a, b in ((dq, dq_r), (dk, dk_r), (dv, dv_r)):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-12)
    if with_sink:
        np.testing.assert_allclose(ds, ds_r, rtol=1e-9, atol=1e-12)


def test_dense_attention_matches_brute_force_loops():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((1, 2, 6, 4)) for _ in range(3))
    sink = np.array([[[[0.3]], [[-0.2]]]])
    np.testing.assert_allclose(OA.dense_forward(q, k, v, sink), CF.attention_brute_force(q, k, v, sink),
                               rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("bf16", 2e-2)])
@pytest.mark.parametrize("shifted", [False, True])
def test_kernel_restatement_matches_dense(dtype, tol, shifted):
    B, H, T, D = 1, 2, 96, 64
    q, k, v, do, sink = attention_inputs(B, H, T, D, seed=3, dtype=dtype)
    q_s, sk, alpha = OA.prologue(q, sink, dtype=dtype)
    o, stat, op = OA.kernel_forward(q_s, k, v, sk, dtype=dtype, shifted=shifted)
    o_res = op if shifted else o
    dq_s, dk, dv, di, dbeta, dq = OA.kernel_backward(q_s, k, v, sk, o_res, stat, do, alpha=alpha, dtype=dtype,
                                                      shifted=shifted, di_from_weights=shifted and dtype == "bf16")
    o_ref = OA.dense_forward(q, k, v, sink)
    dq_r, dk_r, dv_r, ds_r = OA.dense_backward(q, k, v, sink, do)
    assert rel_l2(o, o_ref) < tol
    assert rel_l2(dq, dq_r) < tol and rel_l2(dk, dk_r) < tol and rel_l2(dv, dv_r) < tol
    assert rel_l2(dbeta / 8.0, ds_r.reshape(-1)) < tol


@pytest.mark.parametrize("dtype,tol", [("f32", 2e-6), ("bf16", 1e-2)])
def test_shifted_di_from_weights_is_the_output_dot(dtype, tol):
    """di = sum_j p_ij dP_ij (the HIP bf16 fallback's rule) against the reference's
    di = <dO_i, o_i> over the f32 output (flash.py:633 with precise_output): equal up to f32
    rounding in f32, and up to the bf16 rounding of the weights before PV in bf16."""
    q, k, v, do, sink = attention_inputs(1, 2, 80, 64, seed=6, dtype=dtype, qk_norm=False, scale=3.0)
    q_s, sk, alpha = OA.prologue(q, sink, dtype=dtype)
    o, stat, op = OA.kernel_forward(q_s, k, v, sk, dtype=dtype, shifted=True)
    di_out = OA.kernel_backward(q_s, k, v, sk, op, stat, do, dtype=dtype, shifted=True)[3]
    di_w = OA.kernel_backward(q_s, k, v, sk, op, stat, do, dtype=dtype, shifted=True, di_from_weights=True)[3]
    assert rel_l2(di_w, di_out) < tol
    assert rel_l2(di_w, np.sum(do.astype(np.float64) * OA.dense_forward(q, k, v, sink), -1)) < max(tol, 1e-5)


def test_shifted_di_from_weights_centres_equal_keys():
    """With every score equal the weights are uniform and sum_j p_ij (dP_ij - di_i) = 0, so the
    exact dq is 0. Without the bf16 rounding of the score gradients (f32) the weights rule
    leaves only f32 rounding in dq_s, two orders below what a di off by 2^-12 leaves."""
    shape = (1, 1, 64, 64)
    q = np.full(shape, np.sqrt(1000.0), np.float32)
    v = attention_inputs(1, 1, 64, 64, seed=7, dtype="f32")[2]
    do = np.ones(shape, np.float32)
    q_s, _, alpha = OA.prologue(q, None, dtype="f32")
    o, stat, op = OA.kernel_forward(q_s, q, v, None, dtype="f32", shifted=True)
    dq_w = OA.kernel_backward(q_s, q, v, None, op, stat, do, dtype="f32", shifted=True, di_from_weights=True)[0]
    dq_bad = OA.kernel_backward(q_s, q, v, None, op * np.float32(1 + 2.0 ** -12), stat, do, dtype="f32",
                                shifted=True)[0]
    assert np.linalg.norm(dq_w) < 1e-2 * np.linalg.norm(dq_bad)


@pytest.mark.parametrize("case", ["scale4.5", "scale6", "tail+", "tail-"])
@pytest.mark.parametrize("D", [64, 128])
def test_shifted_di_rules_gap_is_bounded(case, D):
    """The bf16 shifted fallback's two di rules side by side: the reference's
    di = <dO, o_precise> over the f32 output (flash.py:73, 322, 852) and the HIP kernels'
    di = sum_j p_ij dP_ij from the weights. Guard-tripping random inputs (q, k x 4.5 or 6):
    the gradients of the two differ by at most 5e-3 relative L2 (measured about 2e-3, the
    size of one bf16 rounding), well inside what either keeps from the float64 dense
    gradients. The reference's bf16 guarded tails (q = k = +-sqrt(1000),
    test_flash_kernel_tpu.py:238-255, whose exact dq is 0): the gradients of the two rules
    differ by less than 1e-3 of the reference test's 0.012 tolerance."""
    if case.startswith("scale"):
        q, k, v, do, sink = attention_inputs(2, 2, 200, D, seed=9, dtype="bf16", scale=float(case[5:]))
    else:
        shape = (1, 2, 256, D)
        q = np.full(shape, np.sqrt(1000.0), np.float32)
        k = q * (1.0 if case == "tail+" else -1.0)
        rng = np.random.default_rng(3)
        v, do = (round_bf16(rng.standard_normal(shape).astype(np.float32)) for _ in range(2))
        sink = np.zeros((1, 2, 1, 1), np.float32)
    ref = OA.flash_attention_oracle(q, k, v, sink, do, dtype="bf16", di_rule="precise_output")
    hip = OA.flash_attention_oracle(q, k, v, sink, do, dtype="bf16", di_rule="weights")
    assert not ref["in_range"] and not hip["in_range"]
    dense = dict(zip(("dq", "dk", "dv", "dsink"), OA.dense_backward(q, k, v, sink, do)))
    for name in ("dq", "dk", "dv", "dsink"):
        a, b = ref[name].astype(np.float64), hip[name].astype(np.float64)
        if case.startswith("scale"):
            gap = rel_l2(b, a)
            assert gap < 5e-3, (name, gap)
            assert gap < max(rel_l2(a, dense[name]), rel_l2(b, dense[name])) + 1e-3, name
        else:
            assert np.max(np.abs(a - b)) < 0.012 * 1e-3, name


def test_planted_mistakes_fail_the_pins():
    """A dropped sink term or a wrong slope in a restatement is caught by the closed form."""
    q, k, v, do, sink = attention_inputs(1, 2, 48, 64, seed=4, dtype="f32", sink_std=1.0)
    q_s, sk, alpha = OA.prologue(q, sink, dtype="f32")
    o, stat, _ = OA.kernel_forward(q_s, k, v, None, dtype="f32")  # sink dropped
    assert rel_l2(o, OA.dense_forward(q, k, v, sink)) > 1e-3
    o, stat, _ = OA.kernel_forward(q_s, k, v, sk, dtype="f32")
    dq_s, dk, dv, di, dbeta, dq = OA.kernel_backward(q_s, k, v, sk, o, stat, do, n=8, alpha=alpha, dtype="f32")
    dq_r = OA.dense_backward(q, k, v, sink, do)[0]
    assert rel_l2(dq, dq_r) > 1e-2   # slope n=8 instead of 16


def test_guard_predicate():
    q, k, v, do, sink = attention_inputs(1, 2, 64, 128, seed=5, dtype="f32")
    q_s, sk, _ = OA.prologue(q, sink, dtype="f32")
    assert OA.guard_in_range(q_s, k, v, sk)
    big = np.full_like(q, math.sqrt(1000.0))
    q_s2, _, _ = OA.prologue(big, sink, dtype="f32")
    assert not OA.guard_in_range(q_s2, big, v, sk)
    assert not OA.guard_in_range(q_s, k, v * 1e9, sk)
    assert not OA.guard_in_range(q_s, k, v, sk + 20.0)


@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_gradient_is_exact_nll_gradient(n, c):
    rng = np.random.default_rng(1)
    h = rng.standard_normal((6, 5))
    E = rng.standard_normal((11, 5)) * 0.8
    t = np.array([0, 3, 10, 5, 5, 1])
    nll, pt_ref, dh_ref, dE_ref = CF.head_closed_form(h, E, t, n=n, c=c)
    obj, pt = OH.dense_forward(h, E, t, n=n, c=c)
    np.testing.assert_allclose(pt, pt_ref, rtol=1e-9)
    np.testing.assert_allclose(obj, np.mean(1 - pt_ref), rtol=1e-12)
    dh, dE = OH.dense_backward(h, E, t, 1.0, n=n, c=c)
    np.testing.assert_allclose(dh, dh_ref, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dE, dE_ref, rtol=1e-9, atol=1e-12)


def test_head_kernel_restatement_matches_dense():
    h, E, t = head_inputs(256, 64, 300, seed=3, e_std=0.15)
    stat, zt, pt, obj = OH.kernel_forward(h, E, t)
    obj_r, pt_r = OH.dense_forward(h, E, t)
    np.testing.assert_allclose(obj, obj_r, rtol=1e-5)
    np.testing.assert_allclose(pt, pt_r, rtol=1e-4)
    dh, dE = OH.kernel_backward(h, E, t, stat)
    dh_r, dE_r = OH.dense_backward(h, E, t)
    assert rel_l2(dh, dh_r) < 1e-2 and rel_l2(dE, dE_r) < 1e-2


@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_kernel_restatement_f32_matches_dense(n, c):
    """With f32 hidden states nothing is rounded to bf16 (the logit gradient is stored in the
    hidden dtype, fused_head.py:145): the f32 restatement meets the dense float64 head at f32
    precision, and planting a bf16 rounding of the logit gradient breaks that."""
    rng = np.random.default_rng(40 + n)
    h = rng.standard_normal((192, 96)).astype(np.float32)
    E = (rng.standard_normal((517, 96)) * 0.15).astype(np.float32)
    t = rng.integers(0, 517, 192).astype(np.int32)
    stat, zt, pt, obj = OH.kernel_forward(h, E, t, n=n, c=c, dtype="f32")
    obj_r, pt_r = OH.dense_forward(h, E, t, n=n, c=c)
    np.testing.assert_allclose(obj, obj_r, rtol=1e-6)
    np.testing.assert_allclose(pt, pt_r, rtol=1e-5)
    dh, dE = OH.kernel_backward(h, E, t, stat, 0.7, n=n, c=c, dtype="f32", e_dtype="f32")
    dh_r, dE_r = OH.dense_backward(h, E, t, 0.7, n=n, c=c)
    assert rel_l2(dh, dh_r) < 2e-6 and rel_l2(dE, dE_r) < 2e-6
    dh_b, _ = OH.kernel_backward(h, E, t, stat, 0.7, n=n, c=c, dtype="f32", e_dtype="f32", dz_dtype="bf16")
    assert rel_l2(dh_b, dh_r) > 1e-4


def test_eval_logprob_is_log_of_lean_pt():
    """evaluation.logprob_from_logits == log(pt) of the lean likelihood (test_components.py:56),
    and == a per-token brute-force log-softmax loop; argmax == the largest logit."""
    import math
    from helpers import head_inputs
    h, E, t = head_inputs(24, 32, 50, seed=13, e_std=0.5)
    lp, am, z = OH.eval_logprob(h, E, t, n=8, c=2.0)
    _, pt = OH.dense_forward(h, E, t, n=8, c=2.0)
    np.testing.assert_allclose(lp, np.log(pt), rtol=1e-9)
    for i in range(len(t)):
        a = [8 * math.asinh(float(zz) / 2.0) for zz in z[i]]
        mx = max(a)
        ref = a[t[i]] - (mx + math.log(sum(math.exp(x - mx) for x in a)))
        assert abs(lp[i] - ref) < 1e-9
        assert am[i] == max(range(len(a)), key=lambda j: (z[i][j], -j))
