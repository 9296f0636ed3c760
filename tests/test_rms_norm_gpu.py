"""GPU parity of the final RMS norm (model.py:208; algebraic.py:76-83) and its VJP against the
oracle (oracle/prologue.py rms_norm / rms_norm_vjp, pinned to float64 closed forms and torch
autograd by tests/test_prologue_oracle.py), and of the norm composed with the fused head.

Bars: y and dx relative L2 1e-4 (identical rounding points; only the f32 summation order of
the row statistics differs), tau 1e-6, dgain 1e-5 (sums over every row).
"""

import numpy as np
import pytest

from helpers import head_inputs, rel_l2
from oracle import head as OH
from oracle import prologue as OP
from oracle.numerics import round_bf16

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _norm():
    from algebraic_amd.kernels.norm import rms_norm
    return rms_norm


@pytest.mark.parametrize("rows,d", [(300, 768), (257, 2048), (64, 72), (130, 4096), (16384, 2048)])
@pytest.mark.parametrize("gain", [True, False])
def test_rms_norm_matches_oracle(rows, d, gain):
    rng = np.random.default_rng(rows + d)
    x = round_bf16((rng.standard_normal((rows, d)) * 2.5).astype(np.float32))
    dy = round_bf16(rng.standard_normal((rows, d)).astype(np.float32))
    g = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32) if gain else None
    print(f"[rms_norm] {rows}x{d} gain={gain}", flush=True)
    tx = torch.tensor(x, device="cuda").to(torch.bfloat16).requires_grad_(True)
    tg = None if g is None else torch.tensor(g, device="cuda", requires_grad=True)
    y = _norm()(tx, tg)
    y.backward(torch.tensor(dy, device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    y_ref, tau = OP.rms_norm(x, g, 1e-5, "bf16")
    dx_ref, dg_ref = OP.rms_norm_vjp(x, g, tau, dy, "bf16")
    errs = {"y": rel_l2(y.detach().float().cpu().numpy(), y_ref), "dx": rel_l2(tx.grad.float().cpu().numpy(), dx_ref)}
    if g is not None:
        errs["dgain"] = rel_l2(tg.grad.cpu().numpy(), dg_ref)
    print(f"  {errs}", flush=True)
    assert errs["y"] < 1e-4 and errs["dx"] < 1e-4 and errs.get("dgain", 0) < 1e-5, errs


def test_final_norm_then_head_matches_oracle():
    """x -> rms_norm(x, g) -> fused head (residual schedule): objective, telemetry and the
    gradients w.r.t. x, g and E against the oracle chain (norm, kernel-faithful head, norm VJP)."""
    from algebraic_amd.kernels.fused_head import fused_head
    N, d, V = 512, 256, 2304
    rng = np.random.default_rng(3)
    x = round_bf16((rng.standard_normal((N, d)) * 1.7).astype(np.float32))
    g = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    _, E, t = head_inputs(N, d, V, seed=4)
    tx = torch.tensor(x, device="cuda").to(torch.bfloat16).requires_grad_(True)
    tg = torch.tensor(g, device="cuda", requires_grad=True)
    tE = torch.tensor(E, device="cuda").to(torch.bfloat16).requires_grad_(True)
    obj, tel = fused_head(_norm()(tx, tg), tE, torch.tensor(t, device="cuda"), kind="alg_ce", n=8, c=2.0)
    obj.backward()
    torch.cuda.synchronize()
    h, tau = OP.rms_norm(x, g, 1e-5, "bf16")
    stat, _, pt, obj_ref = OH.kernel_forward(h, E, t, n=8, c=2.0)
    dh, dE = OH.kernel_backward(h, E, t, stat, 1.0, n=8, c=2.0)
    dx, dg = OP.rms_norm_vjp(x, g, tau, dh, "bf16")
    errs = {"obj": abs(float(obj.detach()) - float(obj_ref)) / abs(float(obj_ref)),
            "pt": rel_l2(tel.cpu().numpy(), pt), "dx": rel_l2(tx.grad.float().cpu().numpy(), dx),
            "dgain": rel_l2(tg.grad.cpu().numpy(), dg), "dE": rel_l2(tE.grad.float().cpu().numpy(), dE)}
    print(f"  norm+head: {errs}", flush=True)
    assert errs["obj"] < 1e-5 and errs["pt"] < 1e-4 and max(errs["dx"], errs["dgain"], errs["dE"]) < 1e-2, errs
