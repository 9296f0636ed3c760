"""Pins the float32 torch restatement (tests/torch_ref.py) to the NumPy oracle on the CPU.

The full-size GPU parity tests compare the HIP path with tests/torch_ref.py; this file shows
that the torch restatement computes what the oracle computes (every output and gradient, both
input dtypes, with and without a sink), so the full-size comparisons inherit the oracle's pins.
Bars: float32 inputs 1e-5 relative L2; bfloat16 inputs 2e-3 (the two restatements differ only
in f32 summation order, which can move a value across a bf16 rounding boundary).
"""

import numpy as np
import pytest

from helpers import attention_inputs, head_inputs, rel_l2
from oracle import attention as OA
from oracle import head as OH

torch = pytest.importorskip("torch")
import torch_ref  # noqa: E402

TOL = {"bf16": 2e-3, "f32": 1e-5}
TDT = {"bf16": torch.bfloat16, "f32": torch.float32}


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("with_sink", [True, False])
@pytest.mark.parametrize("shape", [(2, 3, 96, 64), (1, 2, 130, 128)])
def test_attention_ref_matches_oracle(shape, dtype, with_sink):
    q, k, v, do, sink = attention_inputs(*shape, seed=5, dtype=dtype, sink=with_sink)
    ref = OA.flash_attention_oracle(q, k, v, sink, do, n=16, c=8.0, dtype=dtype)
    assert ref["in_range"]
    t = lambda a: torch.tensor(a).to(TDT[dtype])
    out = torch_ref.attention(t(q), t(k), t(v), None if sink is None else torch.tensor(sink), t(do),
                              n=16, c=8.0, heads_per_chunk=4)
    names = ["o", "stat", "dq", "dk", "dv", "di"] + (["dsink"] if with_sink else [])
    errs = {name: rel_l2(out[name].numpy().reshape(-1), np.reshape(ref[name], -1)) for name in names}
    bad = {key: val for key, val in errs.items() if not val < TOL[dtype]}
    assert not bad, f"torch restatement differs from the oracle: {bad} (all {errs})"


@pytest.mark.parametrize("shape", [(256, 128, 517), (300, 96, 1000)])
@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_ref_matches_oracle(shape, n, c):
    h, E, tg = head_inputs(*shape, seed=7)
    stat, zt, pt, obj = OH.kernel_forward(h, E, tg, n=n, c=c)
    dh, dE = OH.kernel_backward(h, E, tg, stat, 0.75, n=n, c=c)
    out = torch_ref.head(torch.tensor(h).to(torch.bfloat16), torch.tensor(E).to(torch.bfloat16),
                         torch.tensor(tg), 0.75, n=n, c=c, chunk=128)
    errs = {
        "stat": rel_l2(out["stat"].numpy(), stat), "zt": rel_l2(out["zt"].numpy(), zt),
        "pt": rel_l2(out["pt"].numpy(), pt), "obj": abs(float(out["obj"]) - float(obj)) / abs(float(obj)),
        "dh": rel_l2(out["dh"].numpy(), dh), "dE": rel_l2(out["dE"].numpy(), dE),
    }
    bad = {key: val for key, val in errs.items() if not val < TOL["bf16"]}
    assert not bad, f"torch restatement differs from the oracle: {bad} (all {errs})"


def test_oracle_row_subsets_equal_full_rows():
    """The oracle's row-subset options (used for bounded samples at long T / large N) return
    the rows of the full computation (up to the BLAS blocking of the score products)."""
    q, k, v, do, sink = attention_inputs(1, 2, 200, 64, seed=9)
    q_s, beta, _ = OA.prologue(q, sink, c=8.0)
    o, stat, _ = OA.kernel_forward(q_s, k, v, beta)
    rows = np.array([0, 1, 63, 64, 150, 199])
    o2, stat2, _ = OA.kernel_forward(q_s, k, v, beta, rows=rows, heads=[(0, 1)])
    np.testing.assert_allclose(o2[0, 1, rows], o[0, 1, rows], rtol=1e-2, atol=1e-6)
    assert rel_l2(o2[0, 1, rows], o[0, 1, rows]) < 1e-3
    np.testing.assert_allclose(stat2[0, 1, rows], stat[0, 1, rows], rtol=1e-5)
    assert not np.any(o2[0, 0])

    h, E, tg = head_inputs(300, 64, 700, seed=3)
    stat, *_ = OH.kernel_forward(h, E, tg)
    dh, _ = OH.kernel_backward(h, E, tg, stat)
    toks = np.array([0, 5, 128, 299])
    dh2, _ = OH.kernel_backward(h, E, tg, stat, rows=toks)
    assert rel_l2(dh2[toks], dh[toks]) < 1e-3
    assert not np.any(dh2[1:5])
