"""GPU parity against the committed golden fixtures (tests/golden/*.npz).

The HIP attention (flash_attention mirror, guarded asinh path) and fused head (fused_head
mirror, alg_ce) run on the fixture inputs through the C ABI; outputs and gradients must meet
the north-star bars against the float64 closed forms: bf16 relative L2 2e-2 (attention),
head objective rtol 2e-3, telemetry 2e-2 and gradients 1e-2 (tests/test_fused_head_tpu.py:33-43
in the reference); fp32 attention 1e-5. The final RMS norm and the ALU-GLU block run on their
fixtures at the bf16 bar (2e-2); the streamed eval head on the head fixtures gives log pt of
the closed form (1e-4 absolute) and a float64 argmax.
"""

import glob
import os

import numpy as np
import pytest

from helpers import rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))
HEAD = sorted(glob.glob(os.path.join(GOLDEN, "head_*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def f64(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype,tol", [("bf16", 2e-2), ("f32", 1e-5)])
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_attention_matches_golden(path, dtype, tol):
    from algebraic_amd.kernels.flash import flash_attention
    g = load(path)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    q, k, v = (torch.tensor(g[x], device="cuda").to(tdt).requires_grad_(True) for x in ("q", "k", "v"))
    sink = g.get("sink")
    ts = None if sink is None else torch.tensor(sink, device="cuda", requires_grad=True)
    print(f"golden attention {os.path.basename(path)} {dtype}", flush=True)
    o = flash_attention(q, k, v, ts, kind="asinh", n=int(g["n"]), c=float(g["c"]), range_guard=True,
                        block=q.shape[2])
    o.backward(torch.tensor(g["do"], device="cuda").to(tdt))
    torch.cuda.synchronize()
    got = dict(o=f64(o), dq=f64(q.grad), dk=f64(k.grad), dv=f64(v.grad))
    if ts is not None:
        got["dsink"] = f64(ts.grad)
    errs = {key: rel_l2(val, g[key]) for key, val in got.items()}
    assert all(e < tol for e in errs.values()), errs


@pytest.mark.parametrize("path", HEAD, ids=os.path.basename)
def test_head_matches_golden(path):
    from algebraic_amd.kernels.fused_head import fused_head
    g = load(path)
    h = torch.tensor(g["h"], device="cuda").to(torch.bfloat16).requires_grad_(True)
    E = torch.tensor(g["E"], device="cuda").to(torch.bfloat16).requires_grad_(True)
    t = torch.tensor(g["targets"], device="cuda")
    print(f"golden head {os.path.basename(path)}", flush=True)
    obj, pt = fused_head(h, E, t, kind="alg_ce", n=int(g["n"]), c=float(g["c"]))
    (obj * float(g["g"])).backward()
    torch.cuda.synchronize()
    np.testing.assert_allclose(float(obj.item()), float(g["obj"]), rtol=2e-3, atol=2e-4)
    assert rel_l2(f64(pt), g["pt"]) < 2e-2
    assert rel_l2(f64(h.grad), g["dh"]) < 1e-2
    assert rel_l2(f64(E.grad), g["dE"]) < 1e-2


@pytest.mark.parametrize("path", HEAD, ids=os.path.basename)
def test_head_f32_matches_golden(path):
    """The f32 head (h and E float32; the fixture inputs are bf16-exact, so exact in f32)
    against the float64 closed forms at the f32 bar, 1e-5."""
    from algebraic_amd.kernels.fused_head import fused_head
    g = load(path)
    h = torch.tensor(g["h"], device="cuda", dtype=torch.float32, requires_grad=True)
    E = torch.tensor(g["E"], device="cuda", dtype=torch.float32, requires_grad=True)
    t = torch.tensor(g["targets"], device="cuda")
    print(f"golden head f32 {os.path.basename(path)}", flush=True)
    obj, pt = fused_head(h, E, t, kind="alg_ce", n=int(g["n"]), c=float(g["c"]))
    (obj * float(g["g"])).backward()
    torch.cuda.synchronize()
    np.testing.assert_allclose(float(obj.detach()), float(g["obj"]), rtol=1e-5, atol=1e-8)
    assert rel_l2(f64(pt), g["pt"]) < 1e-5
    assert rel_l2(f64(h.grad), g["dh"]) < 1e-5
    assert rel_l2(f64(E.grad), g["dE"]) < 1e-5


NORM = sorted(glob.glob(os.path.join(GOLDEN, "norm_*.npz")))
FFN = sorted(glob.glob(os.path.join(GOLDEN, "ffn_*.npz")))


@pytest.mark.parametrize("path", NORM, ids=os.path.basename)
def test_norm_matches_golden(path):
    """The HIP final RMS norm (bf16 rows) against the float64 definition: bf16 bar 2e-2."""
    from algebraic_amd.kernels.norm import rms_norm
    z = load(path)
    x = torch.tensor(z["x"], device="cuda").to(torch.bfloat16).requires_grad_(True)
    g = torch.tensor(z["gain"], device="cuda", requires_grad=True) if "gain" in z else None
    print(f"[golden] {os.path.basename(path)}", flush=True)
    y = rms_norm(x, g, eps=float(z["eps"]))
    y.backward(torch.tensor(z["dy"], device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    errs = {"y": rel_l2(f64(y), z["y"]), "dx": rel_l2(f64(x.grad), z["dx"])}
    if g is not None:
        errs["dgain"] = rel_l2(f64(g.grad), z["dgain"])
    assert max(errs.values()) < 2e-2, errs


@pytest.mark.parametrize("path", FFN, ids=os.path.basename)
def test_ffn_matches_golden(path):
    """The HIP ALU-GLU block (fused activation epilogues) against the float64 definition."""
    from algebraic_amd.kernels.ffn import alu_glu_ffn
    z = load(path)
    t = [torch.tensor(z[k], device="cuda").to(torch.bfloat16).requires_grad_(True) for k in ("h2", "w_g", "w_u", "w_d")]
    print(f"[golden] {os.path.basename(path)}", flush=True)
    out = alu_glu_ffn(*t, beta=float(z["beta"]))
    out.backward(torch.tensor(z["dout"], device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    errs = {"out": rel_l2(f64(out), z["out"]), "dh2": rel_l2(f64(t[0].grad), z["dh2"]),
            "dw_g": rel_l2(f64(t[1].grad), z["dw_g"]), "dw_u": rel_l2(f64(t[2].grad), z["dw_u"]),
            "dw_d": rel_l2(f64(t[3].grad), z["dw_d"])}
    assert max(errs.values()) < 2e-2, errs


@pytest.mark.parametrize("path", HEAD, ids=os.path.basename)
def test_eval_head_matches_golden(path):
    """The streamed eval head on the head fixtures: log p(target) = log pt of the float64
    closed form (the identity the reference's scorer relies on), argmax a float64 maximum."""
    from algebraic_amd.kernels.fused_head import head_logprob
    z = load(path)
    h = torch.tensor(z["h"], device="cuda").to(torch.bfloat16)
    E = torch.tensor(z["E"], device="cuda").to(torch.bfloat16)
    print(f"[golden] eval {os.path.basename(path)}", flush=True)
    lp, am = head_logprob(h, E, torch.tensor(z["targets"], device="cuda"), n=int(z["n"]), c=float(z["c"]))
    torch.cuda.synchronize()
    np.testing.assert_allclose(f64(lp), np.log(z["pt"].astype(np.float64)), atol=1e-4)
    logits = z["h"].astype(np.float64) @ z["E"].astype(np.float64).T
    best = logits.max(axis=1)
    got = logits[np.arange(len(best)), am.cpu().numpy()]
    assert np.all(got >= best - 1e-5 * (np.abs(best) + 1))
