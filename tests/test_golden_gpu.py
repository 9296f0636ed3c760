"""GPU parity against the committed golden fixtures (tests/golden/*.npz).

The HIP attention (flash_attention mirror, guarded asinh path) and fused head (fused_head
mirror, alg_ce) run on the fixture inputs through the C ABI; outputs and gradients must meet
the north-star bars against the float64 closed forms: bf16 relative L2 2e-2 (attention),
head objective rtol 2e-3, telemetry 2e-2 and gradients 1e-2 (tests/test_fused_head_tpu.py:33-43
in the reference); fp32 attention 1e-5.
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
