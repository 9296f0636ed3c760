"""GPU parity: HIP algebraic attention (C ABI via the flash_attention mirror) vs the oracle.

Bars (north star; metric = per-tensor relative L2, tests/test_flash_kernel_tpu.py:97-101):
  bf16 inputs: outputs and gradients within 2e-2 of the float64 dense oracle and within
               1e-2 of the cast-faithful kernel restatement;
  fp32 inputs: within 1e-5 of the float64 dense oracle.
Input distributions follow the reference tests (tests/test_flash_kernel_tpu.py:44-123).
"""

import math

import numpy as np
import pytest

from helpers import attention_inputs, rel_l2
from oracle import attention as OA

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

BF16_DENSE, BF16_KERNEL, F32_DENSE = 2e-2, 1e-2, 1e-5


def _flash():
    from algebraic_amd.kernels.flash import flash_attention
    return flash_attention


def _to(x, dtype):
    return torch.tensor(x, device="cuda").to(dtype)


def run_hip(q, k, v, do, sink, dtype, **kw):
    """Forward + backward through flash_attention; returns numpy float64 arrays."""
    flash_attention = _flash()
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    tq, tk, tv = (_to(a, tdt).requires_grad_(True) for a in (q, k, v))
    ts = None if sink is None else torch.tensor(sink, device="cuda", requires_grad=True)
    kw.setdefault("kind", "asinh")
    kw.setdefault("n", 16)
    kw.setdefault("c", 8.0)
    o = flash_attention(tq, tk, tv, ts, **kw)
    o.backward(_to(do, tdt))
    torch.cuda.synchronize()
    f = lambda t: None if t is None else t.detach().float().cpu().numpy().astype(np.float64)
    return f(o), f(tq.grad), f(tk.grad), f(tv.grad), f(None if ts is None else ts.grad)


def check_dense(res, q, k, v, do, sink, tol, n=16, c=8.0):
    o, dq, dk, dv, ds = res
    o_ref = OA.dense_forward(q, k, v, sink, n=n, c=c)
    dq_r, dk_r, dv_r, ds_r = OA.dense_backward(q, k, v, sink, do, n=n, c=c)
    errs = {"o": rel_l2(o, o_ref), "dq": rel_l2(dq, dq_r), "dk": rel_l2(dk, dk_r), "dv": rel_l2(dv, dv_r)}
    if sink is not None:
        errs["dsink"] = rel_l2(ds, ds_r)
    bad = {key: val for key, val in errs.items() if not val < tol}
    assert not bad, f"dense parity failed {bad} (all {errs})"
    return errs


CASES = [  # (B, H, T, D)
    (1, 2, 64, 64),
    (2, 3, 100, 64),     # ragged T, not a tile multiple
    (1, 2, 256, 128),
    (1, 1, 33, 128),     # T just past one 32-row block
    (2, 2, 384, 64),
    (1, 2, 1, 64),       # one position
    (2, 1, 2, 128),      # two positions
    (1, 3, 17, 64),      # a partial first tile
]


@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("with_sink", [True, False])
def test_guarded_bf16_matches_oracle(shape, with_sink):
    B, H, T, D = shape
    q, k, v, do, sink = attention_inputs(B, H, T, D, seed=3, sink=with_sink)
    res = run_hip(q, k, v, do, sink, "bf16", range_guard=True, block=T)
    if T == 1 and not with_sink:
        # One key and no sink: p = 1, o = v, and every exact gradient of q is 0 (the score
        # gradient p (dP - di) vanishes); di from the bf16 output leaves rounding noise, so
        # dq is held to an absolute bar on the scale of dO . k, the rest to the usual ones.
        assert np.abs(res[1]).max() <= 1e-2 * np.abs(do).max() * np.abs(k).max()
        o_ref = OA.dense_forward(q, k, v, sink)
        _, dk_r, dv_r, _ = OA.dense_backward(q, k, v, sink, do)
        assert rel_l2(res[0], o_ref) < BF16_DENSE and rel_l2(res[3], dv_r) < BF16_DENSE
        assert np.abs(res[2]).max() <= 1e-2 * np.abs(do).max() * np.abs(q).max()
        return
    check_dense(res, q, k, v, do, sink, BF16_DENSE)
    ref = OA.flash_attention_oracle(q, k, v, sink, do, dtype="bf16")
    assert ref["in_range"]
    assert rel_l2(res[0], ref["o"]) < BF16_KERNEL
    for got, key in zip(res[1:4], ("dq", "dk", "dv")):
        assert rel_l2(got, ref[key]) < BF16_KERNEL, key
    if with_sink:
        assert rel_l2(res[4], ref["dsink"]) < BF16_KERNEL


@pytest.mark.parametrize("shape", [(1, 2, 64, 64), (2, 3, 100, 64), (1, 2, 160, 128)])
@pytest.mark.parametrize("with_sink", [True, False])
def test_guarded_fp32_matches_dense(shape, with_sink):
    B, H, T, D = shape
    q, k, v, do, sink = attention_inputs(B, H, T, D, seed=5, dtype="f32", sink=with_sink)
    res = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=T)
    check_dense(res, q, k, v, do, sink, F32_DENSE)


@pytest.mark.parametrize("shape", [(8, 16, 256, 64), (8, 16, 200, 64)])
@pytest.mark.parametrize("with_sink", [True, False])
def test_guarded_fp32_two_way_key_split(shape, with_sink):
    """f32 D = 64 grids of at least 512 two-way workgroups (B H ceil(T/64) >= 512) split each
    row's keys over two waves (64 queries per workgroup); smaller grids, as in the other f32
    cases, split them four ways. Both against the dense float64 reference at the f32 bar."""
    B, H, T, D = shape
    q, k, v, do, sink = attention_inputs(B, H, T, D, seed=7, dtype="f32", sink=with_sink)
    res = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=T)
    check_dense(res, q, k, v, do, sink, F32_DENSE)


def test_config1_fp32_125m_shape():
    """B=2, H=12, T=1024, D=64 fp32 forward (+ backward) at 1e-5."""
    q, k, v, do, sink = attention_inputs(2, 12, 1024, 64, seed=11, dtype="f32")
    res = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=512)
    check_dense(res, q, k, v, do, sink, F32_DENSE)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_unnormalised_inputs_scale_15(dtype):
    """Q/K ~ N(0,1)*1.5 without QK norm (tests/test_flash_kernel_tpu.py:44-70)."""
    q, k, v, do, sink = attention_inputs(2, 3, 128, 64, seed=7, dtype=dtype, qk_norm=False, scale=1.5,
                                         sink_std=0.5)
    res = run_hip(q, k, v, do, sink, dtype, range_guard=True, block=128)
    check_dense(res, q, k, v, do, sink, BF16_DENSE if dtype == "bf16" else 1e-4)


@pytest.mark.parametrize("score_sign", [-1.0, 1.0])
@pytest.mark.parametrize("with_sink", [False, True])
@pytest.mark.parametrize("magnitude", [1000.0, 1e7])
def test_guarded_attention_tail(score_sign, with_sink, magnitude):
    """Out-of-range inputs take the shifted branch (tests/test_flash_kernel_tpu.py:104-123)."""
    shape = (1, 1, 256, 64)
    q = np.full(shape, math.sqrt(magnitude), np.float32)
    k = q * score_sign
    v = np.random.default_rng(29).standard_normal(shape).astype(np.float32)
    do = np.ones(shape, np.float32)
    sink = np.zeros((1,), np.float32) if with_sink else None
    res = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=128)
    o_ref = OA.dense_forward(q, k, v, sink)
    assert np.isfinite(res[0]).all()
    np.testing.assert_allclose(res[0], o_ref, atol=2e-3, rtol=2e-3)
    assert all(np.isfinite(g).all() for g in res[1:4])


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_unguarded_default_variant(dtype):
    """range_guard=False: the clipped unshifted default of make_variant (flash.py:749-754)."""
    q, k, v, do, sink = attention_inputs(1, 2, 192, 64, seed=9, dtype=dtype)
    res = run_hip(q, k, v, do, sink, dtype, range_guard=False, block=64)
    check_dense(res, q, k, v, do, sink, BF16_DENSE if dtype == "bf16" else F32_DENSE)


@pytest.mark.parametrize("fast", [True, False])
def test_explicit_shift_variant(fast):
    """shift=True accumulation with fast or stable rho (flash.py:235-259)."""
    q, k, v, do, sink = attention_inputs(1, 2, 128, 64, seed=13, dtype="f32")
    res = run_hip(q, k, v, do, sink, "f32", shift=True, fast_rho=fast, block=64)
    check_dense(res, q, k, v, do, sink, 1e-5)


def test_causality_future_keys_do_not_leak():
    """Perturbing keys/values after row i leaves rows <= i unchanged (test_e2e_acceptance.py:590-594)."""
    q, k, v, do, sink = attention_inputs(1, 2, 256, 128, seed=17)
    a = run_hip(q, k, v, do, sink, "bf16", range_guard=True, block=256)[0]
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 150:] = np.flip(k2[:, :, 150:], axis=-1)
    v2[:, :, 150:] *= -3.0
    b = run_hip(q, k2, v2, do, sink, "bf16", range_guard=True, block=256)[0]
    np.testing.assert_array_equal(a[:, :, :150], b[:, :, :150])
    assert not np.array_equal(a[:, :, 150:], b[:, :, 150:])


def test_rows_sum_to_one_minus_sink_mass():
    """With v = 1 every output row equals 1 - sink mass (normalisation invariant)."""
    B, H, T, D = 2, 4, 512, 64
    q, k, _, do, sink = attention_inputs(B, H, T, D, seed=19, dtype="f32")
    v = np.ones((B, H, T, D), np.float32)
    o = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=512)[0]
    p, psink, _ = OA._dense_probs(q.astype(np.float64), k.astype(np.float64), 16, 8.0,
                                  OA._sink_vector(sink, H))
    np.testing.assert_allclose(o[..., 0], 1.0 - psink, rtol=2e-6, atol=2e-6)


# Head widths other than the built 64 and 128 (the reference's generic kernels take any D,
# flash.py:189-326): the mirror runs them zero-padded to the next built width with c and the
# sink rescaled so that alpha = 1/(sqrt(D) c) and sink/c are the logical width's.
@pytest.mark.parametrize("D", [32, 48, 80, 96])
@pytest.mark.parametrize("with_sink", [True, False])
def test_guarded_bf16_other_head_dims(D, with_sink):
    q, k, v, do, sink = attention_inputs(2, 3, 100, D, seed=61 + D, sink=with_sink)
    print(f"[head_dim] bf16 D={D} sink={with_sink}", flush=True)
    res = run_hip(q, k, v, do, sink, "bf16", range_guard=True, block=100)
    assert res[0].shape[-1] == D
    check_dense(res, q, k, v, do, sink, BF16_DENSE)
    ref = OA.flash_attention_oracle(q, k, v, sink, do, dtype="bf16")
    assert ref["in_range"]
    for got, key in zip(res, ("o", "dq", "dk", "dv", "dsink")):
        if got is not None and key in ref:
            assert rel_l2(got, ref[key]) < BF16_KERNEL, key


@pytest.mark.parametrize("D", [16, 96])
def test_guarded_fp32_other_head_dims(D):
    q, k, v, do, sink = attention_inputs(1, 2, 160, D, seed=67 + D, dtype="f32")
    print(f"[head_dim] f32 D={D}", flush=True)
    res = run_hip(q, k, v, do, sink, "f32", range_guard=True, block=160)
    check_dense(res, q, k, v, do, sink, F32_DENSE)


@pytest.mark.parametrize("variant", ["shifted_fallback", "clipped", "bthd"])
def test_other_head_dim_variants(variant):
    """D = 96 on the guard's shifted fallback (q, k x 4.5), the clipped unguarded default and
    the (B, T, H, D) projection layout."""
    D = 96
    scale = 4.5 if variant == "shifted_fallback" else 1.0
    q, k, v, do, sink = attention_inputs(2, 2, 128, D, seed=73, scale=scale)
    print(f"[head_dim] D={D} {variant}", flush=True)
    if variant == "bthd":
        from algebraic_amd.kernels.flash import flash_attention
        tr = lambda a: np.ascontiguousarray(np.transpose(a, (0, 2, 1, 3)))
        tq, tk, tv = (_to(tr(a), torch.bfloat16).requires_grad_(True) for a in (q, k, v))
        ts = torch.tensor(sink, device="cuda", requires_grad=True)
        o = flash_attention(tq, tk, tv, ts, kind="asinh", n=16, c=8.0, range_guard=True, layout="bthd")
        o.backward(_to(tr(do), torch.bfloat16))
        back = lambda t: np.transpose(t.detach().float().cpu().numpy().astype(np.float64), (0, 2, 1, 3))
        res = (back(o), back(tq.grad), back(tk.grad), back(tv.grad), ts.grad.cpu().numpy().astype(np.float64))
    else:
        kw = dict(range_guard=True) if variant == "shifted_fallback" else dict(range_guard=False)
        res = run_hip(q, k, v, do, sink, "bf16", block=128, **kw)
    check_dense(res, q, k, v, do, sink, BF16_DENSE)
    if variant == "shifted_fallback":
        ref = OA.flash_attention_oracle(q, k, v, sink, do, dtype="bf16")
        assert not ref["in_range"]
        for got, key in zip(res, ("o", "dq", "dk", "dv", "dsink")):
            assert rel_l2(got, ref[key]) < BF16_KERNEL, key
