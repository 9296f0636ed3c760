"""The oracle against the committed golden fixtures (CPU).

Fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) hold bf16-exact inputs and
the float64 closed-form outputs of softmax attention over n*asinh(s/c) logits with a sink column
and of the algebraic head's true NLL (tests/test_components.py:27-56 in the reference), stored
as float32. The dense float64 oracle must reproduce them to float32 storage precision; the
cast-faithful kernel restatements must meet the north-star bars (bf16 2e-2, fp32 1e-5). The
final RMS norm and ALU-GLU fixtures hold their float64 definitions (algebraic.py:76-103,
model.py:185-193) and gradients; the oracle meets them the same way.
"""

import glob
import os

import numpy as np
import pytest

from helpers import rel_l2
from oracle import attention as OA
from oracle import head as OH

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))
HEAD = sorted(glob.glob(os.path.join(GOLDEN, "head_*.npz")))
STORE = 2e-6  # float32 storage of float64 results


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(ATTN) >= 2 and len(HEAD) >= 2


@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_dense_attention_oracle_matches_golden(path):
    g = load(path)
    n, c = int(g["n"]), float(g["c"])
    sink = g.get("sink")
    o = OA.dense_forward(g["q"], g["k"], g["v"], sink, n=n, c=c)
    dq, dk, dv, ds = OA.dense_backward(g["q"], g["k"], g["v"], sink, g["do"], n=n, c=c)
    assert rel_l2(o, g["o"]) < STORE
    assert rel_l2(dq, g["dq"]) < STORE
    assert rel_l2(dk, g["dk"]) < STORE
    assert rel_l2(dv, g["dv"]) < STORE
    if sink is not None:
        assert rel_l2(ds, g["dsink"]) < STORE


@pytest.mark.parametrize("dtype,tol", [("bf16", 2e-2), ("f32", 1e-5)])
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_kernel_attention_oracle_within_bar_of_golden(path, dtype, tol):
    g = load(path)
    sink = g.get("sink")
    res = OA.flash_attention_oracle(g["q"], g["k"], g["v"], sink, g["do"], n=int(g["n"]), c=float(g["c"]),
                                    dtype=dtype)
    for key in ("o", "dq", "dk", "dv") + (("dsink",) if sink is not None else ()):
        assert rel_l2(res[key], g[key]) < tol, key


@pytest.mark.parametrize("path", HEAD, ids=os.path.basename)
def test_dense_head_oracle_matches_golden(path):
    g = load(path)
    n, c = int(g["n"]), float(g["c"])
    obj, pt = OH.dense_forward(g["h"], g["E"], g["targets"], n=n, c=c)
    dh, dE = OH.dense_backward(g["h"], g["E"], g["targets"], float(g["g"]), n=n, c=c)
    np.testing.assert_allclose(obj, g["obj"], rtol=1e-9)
    assert rel_l2(pt, g["pt"]) < STORE
    assert rel_l2(dh, g["dh"]) < STORE
    assert rel_l2(dE, g["dE"]) < STORE


@pytest.mark.parametrize("path", HEAD, ids=os.path.basename)
def test_kernel_head_oracle_within_bar_of_golden(path):
    g = load(path)
    n, c = int(g["n"]), float(g["c"])
    stat, zt, pt, obj = OH.kernel_forward(g["h"], g["E"], g["targets"], n=n, c=c)
    dh, dE = OH.kernel_backward(g["h"], g["E"], g["targets"], stat, float(g["g"]), n=n, c=c)
    np.testing.assert_allclose(obj, g["obj"], rtol=2e-3, atol=2e-4)
    assert rel_l2(pt, g["pt"]) < 2e-2
    assert rel_l2(dh, g["dh"]) < 1e-2
    assert rel_l2(dE, g["dE"]) < 1e-2


NORM = sorted(glob.glob(os.path.join(GOLDEN, "norm_*.npz")))
FFN = sorted(glob.glob(os.path.join(GOLDEN, "ffn_*.npz")))


def test_neighbour_fixtures_present():
    assert len(NORM) >= 2 and len(FFN) >= 2


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("bf16", 2e-2)])
@pytest.mark.parametrize("path", NORM, ids=os.path.basename)
def test_norm_oracle_matches_golden(path, dtype, tol):
    """oracle/prologue.py rms_norm and rms_norm_vjp against the float64 definition
    (algebraic.py:76-83): f32 to storage precision, the bf16 cast-faithful form within 2e-2."""
    from oracle import prologue as OP
    z = load(path)
    g = z.get("gain")
    y, tau = OP.rms_norm(z["x"], g, float(z["eps"]), dtype)
    dx, dg = OP.rms_norm_vjp(z["x"], g, tau, z["dy"], dtype)
    errs = {"y": rel_l2(y, z["y"]), "dx": rel_l2(dx, z["dx"])}
    if g is not None:
        errs["dgain"] = rel_l2(dg, z["dgain"])
    assert max(errs.values()) < tol, errs


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("bf16", 2e-2)])
@pytest.mark.parametrize("path", FFN, ids=os.path.basename)
def test_ffn_oracle_matches_golden(path, dtype, tol):
    """oracle/ffn.py against the float64 ALU-GLU block (model.py:185-193, algebraic.py:84-103)."""
    from oracle import ffn as OF
    z = load(path)
    beta = float(z["beta"])
    out, *_ = OF.ffn_forward(z["h2"], z["w_g"], z["w_u"], z["w_d"], beta, dtype)
    dh2, dw_g, dw_u, dw_d, _, _ = OF.ffn_backward(z["h2"], z["w_g"], z["w_u"], z["w_d"], z["dout"], beta, dtype)
    errs = {"out": rel_l2(out, z["out"]), "dh2": rel_l2(dh2, z["dh2"]), "dw_g": rel_l2(dw_g, z["dw_g"]),
            "dw_u": rel_l2(dw_u, z["dw_u"]), "dw_d": rel_l2(dw_d, z["dw_d"])}
    assert max(errs.values()) < tol, errs
