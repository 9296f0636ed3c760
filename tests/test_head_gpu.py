"""GPU parity: HIP fused algebraic head (fused_head mirror over the C ABI) vs the oracle.

Bars follow the reference's head tests (tests/test_fused_head_tpu.py:33-43, 66-70):
objective rtol 2e-3, telemetry rtol 2e-2, gradients relative L2 < 1e-2 against the float64
dense oracle (and < 1e-2 against the cast-faithful kernel restatement).
"""

import numpy as np
import pytest

from helpers import head_inputs, rel_l2
from oracle import head as OH

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def run_hip(h, E, t, n=8, c=2.0, e_dtype=torch.bfloat16, g=1.0):
    from algebraic_amd.kernels.fused_head import fused_head
    th = torch.tensor(h, device="cuda").to(torch.bfloat16).requires_grad_(True)
    tE = torch.tensor(E, device="cuda").to(e_dtype).requires_grad_(True)
    tt = torch.tensor(t, device="cuda")
    obj, tel = fused_head(th, tE, tt, kind="alg_ce", n=n, c=c)
    (obj * g).backward()
    torch.cuda.synchronize()
    f = lambda x: x.detach().float().cpu().numpy().astype(np.float64)
    return float(obj.item()), f(tel), f(th.grad), f(tE.grad)


CASES = [  # (N, d, V)
    (256, 128, 300),
    (256, 256, 4096),
    (128, 128, 517),     # ragged vocab
    (384, 256, 1000),    # token count not a 256 multiple
    (100, 128, 260),     # N < 128 (single ragged token tile)
    (512, 512, 2304),    # several k-step pairs in every product
    (256, 72, 333),      # d not a multiple of the k step or of a tile
    (1, 8, 300),         # one token, the narrowest rows
    (5, 16, 513),        # a few tokens, a vocabulary just past two 256-row chunks
]


@pytest.fixture(params=["residual", "recompute", "streamed"])
def schedule(request, monkeypatch):
    """The three backward schedules; "streamed" with 256-row vocabulary chunks, so every
    case runs several chunks (a ragged last one where V % 256 != 0)."""
    from algebraic_amd.kernels import fused_head as FH
    monkeypatch.setattr(FH, "SCHEDULE", request.param)
    if request.param == "streamed":
        monkeypatch.setattr(FH, "VOCAB_CHUNK", 256)
    return request.param


@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("n,c", [(8, 2.0), (16, 16.0)])
def test_head_matches_dense(shape, n, c, schedule):
    N, d, V = shape
    h, E, t = head_inputs(N, d, V, seed=4, e_std=0.15)
    obj, pt, dh, dE = run_hip(h, E, t, n=n, c=c)
    obj_r, pt_r = OH.dense_forward(h, E, t, n=n, c=c)
    dh_r, dE_r = OH.dense_backward(h, E, t, 1.0, n=n, c=c)
    np.testing.assert_allclose(obj, obj_r, rtol=2e-3, atol=2e-4)
    np.testing.assert_allclose(pt, pt_r, rtol=2e-2, atol=2e-4)
    assert rel_l2(dh, dh_r) < 1e-2
    assert rel_l2(dE, dE_r) < 1e-2
    stat, zt, pt_k, obj_k = OH.kernel_forward(h, E, t, n=n, c=c)
    dh_k, dE_k = OH.kernel_backward(h, E, t, stat, 1.0, n=n, c=c)
    assert rel_l2(dh, dh_k) < 1e-2
    assert rel_l2(dE, dE_k) < 1e-2


def test_head_model_init_scale_and_f32_embedding(schedule):
    """E ~ N(0, 0.02) as the model initialises it, stored f32 (dE returned in f32)."""
    N, d, V = 256, 256, 2048
    h, E, t = head_inputs(N, d, V, seed=6, e_std=0.02)
    obj, pt, dh, dE = run_hip(h, E, t, e_dtype=torch.float32, g=0.5)
    obj_r, pt_r = OH.dense_forward(h, E, t)
    dh_r, dE_r = OH.dense_backward(h, E, t, 0.5)
    np.testing.assert_allclose(obj, obj_r, rtol=2e-3, atol=2e-4)
    np.testing.assert_allclose(pt, pt_r, rtol=2e-2, atol=1e-7)
    assert rel_l2(dh, dh_r) < 1e-2
    assert rel_l2(dE, dE_r) < 1e-2


def test_head_gradient_linear_in_cotangent(schedule):
    """dL scales linearly with the objective's cotangent g (scale = g n/c/N)."""
    h, E, t = head_inputs(256, 128, 700, seed=8, e_std=0.1)
    _, _, dh1, dE1 = run_hip(h, E, t, g=1.0)
    _, _, dh2, dE2 = run_hip(h, E, t, g=-2.0)
    assert rel_l2(dh2, -2.0 * dh1) < 1e-2
    assert rel_l2(dE2, -2.0 * dE1) < 1e-2


def test_head_confident_targets_no_cancellation(schedule):
    """p_t near 1: the residual schedule's target entry (w_t - l) r_t keeps dh accurate."""
    N, d, V = 256, 128, 512
    h, E, t = head_inputs(N, d, V, seed=12, e_std=0.02)
    E = E.copy()
    E[t] = h * 3.0      # target rows aligned with the hidden states -> confident predictions
    from oracle.numerics import round_bf16
    E = round_bf16(E)
    obj, pt, dh, dE = run_hip(h, E, t)
    obj_r, pt_r = OH.dense_forward(h, E, t)
    dh_r, dE_r = OH.dense_backward(h, E, t)
    assert np.median(pt_r) > 0.99
    np.testing.assert_allclose(obj, obj_r, rtol=2e-2, atol=2e-4)
    assert rel_l2(dh, dh_r) < 2e-2
    assert rel_l2(dE, dE_r) < 2e-2


@pytest.mark.parametrize("N,d,V,n,c", [(1024, 256, 4096, 16, 16.0), (1024, 256, 32768, 16, 16.0),
                                       (1024, 256, 4096, 8, 2.0), (384, 256, 1000, 16, 16.0)])
def test_residual_block_every_entry(N, d, V, n, c):
    """Every entry of the forward's residual block U (token-major, Npad x Vp bf16) against
    bf16(w r), target entries bf16((w_t - l) r_t), on two calls in a row. A relative L2 bar on
    dh misses a few hundred wrong entries among millions; this compares each one."""
    from algebraic_amd import _lib
    from oracle.numerics import head_clamp, int_pow, round_bf16
    lib, P = _lib.load(), _lib.ptr
    rng = np.random.default_rng(100 + V + n)
    h = round_bf16(rng.standard_normal((N, d)).astype(np.float32))
    E = round_bf16((rng.standard_normal((V, d)) * 0.15).astype(np.float32))
    t = rng.integers(0, V, N).astype(np.int32)
    z = h @ E.T
    x = np.minimum(z * np.float32(1.0 / c), np.float32(head_clamp(V, n)))
    rad = np.float32(1.0) + x * x
    r = np.float32(1.0) / np.sqrt(rad)
    w = int_pow(x + rad * r, n).astype(np.float32)
    l = w.sum(1, dtype=np.float64).astype(np.float32)
    U_ref = w * r
    rows = np.arange(N)
    U_ref[rows, t] = (w[rows, t] - l) * r[rows, t]
    th = torch.tensor(h, device="cuda").to(torch.bfloat16)
    tE = torch.tensor(E, device="cuda").to(torch.bfloat16)
    tt = torch.tensor(t, device="cuda")
    ws_b = lib.alg_head_workspace_size(_lib.DTYPE_BF16, N, d, V, 0)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    Npad, Vp = (N + 255) // 256 * 256, (V + 7) // 8 * 8
    outs = [torch.empty(N, device="cuda") for _ in range(3)] + [torch.empty(1, device="cuda")]
    for call in range(2):
        res = torch.full((lib.alg_head_residual_size(N, d, V),), 0x7F, dtype=torch.uint8, device="cuda")
        _lib.check(lib.alg_head_fwd(_lib.stream_of(th), _lib.DTYPE_BF16, N, d, V, P(th), P(tE), P(tt), n, c, *map(P, outs),
                                    P(res), P(ws), ws_b), "alg_head_fwd")
        torch.cuda.synchronize()
        U = res[:Npad * Vp * 2].view(torch.bfloat16).view(Npad, Vp)[:N, :V].float().cpu().numpy()
        err = np.abs(U - U_ref) / np.abs(U_ref)
        bad = np.argwhere(err > 1e-2)
        assert len(bad) == 0, f"call {call}: {len(bad)} wrong entries, first {bad[:4].tolist()}"
        l_k = res[(Npad * Vp * 2 + 255) // 256 * 256:].view(torch.float32)[:N].cpu().numpy()
        np.testing.assert_allclose(l_k, l, rtol=1e-4)


SPLIT_SHAPE = (2176, 264, 70000)


@pytest.fixture(scope="module")
def split_case():
    N, d, V = SPLIT_SHAPE
    h, E, t = head_inputs(N, d, V, seed=12, e_std=0.15)
    obj_r, _ = OH.dense_forward(h, E, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, E, t, 1.0, n=8, c=2.0)
    return h, E, t, obj_r, dh_r, dE_r


@pytest.mark.parametrize("e_dtype", [torch.bfloat16, torch.float32], ids=["bf16E", "f32E"])
def test_head_de_token_split_tail(e_dtype, schedule, split_case):
    """dE tiles past the last complete round of 256 workgroups are split over the tokens and
    summed by a second kernel (here 274 x 2 = 548 tiles: 512 whole, the 36 tiles of vocabulary
    rows >= 65536 in two unequal ranges of 1152 and 1024 tokens; d = 264 leaves a ragged
    column tile). Gradients against the float64 dense oracle, the split rows also on
    their own, so a lost or doubled token range cannot hide in the whole-matrix norm."""
    h, E, t, obj_r, dh_r, dE_r = split_case
    obj, pt, dh, dE = run_hip(h, E, t, n=8, c=2.0, e_dtype=e_dtype)
    np.testing.assert_allclose(obj, obj_r, rtol=2e-3, atol=2e-4)
    assert rel_l2(dh, dh_r) < 1e-2
    assert rel_l2(dE, dE_r) < 1e-2
    assert rel_l2(dE[65536:], dE_r[65536:]) < 1e-2
    assert rel_l2(dE[65536:, 256:], dE_r[65536:, 256:]) < 1e-2


@pytest.mark.parametrize("chunk", [0, 512, 1280, 4096])
def test_head_streamed_chunks(chunk, monkeypatch):
    """Streamed backward at several chunk sizes (0: the library's default, here one chunk;
    1280: a ragged last chunk of 720 rows) against the float64 dense oracle and the recompute
    schedule: the logit-gradient entries are formed by the same expression, so the gradients
    differ only by the chunked f32 accumulation of dh."""
    from algebraic_amd.kernels import fused_head as FH
    N, d, V = 640, 256, 4560
    h, E, t = head_inputs(N, d, V, seed=33, e_std=0.15)
    print(f"[head streamed] chunk {chunk}", flush=True)
    monkeypatch.setattr(FH, "SCHEDULE", "recompute")
    _, _, dh_rc, dE_rc = run_hip(h, E, t, n=8, c=2.0, g=0.6)
    monkeypatch.setattr(FH, "SCHEDULE", "streamed")
    monkeypatch.setattr(FH, "VOCAB_CHUNK", chunk)
    obj, pt, dh, dE = run_hip(h, E, t, n=8, c=2.0, g=0.6)
    obj_r, _ = OH.dense_forward(h, E, t, n=8, c=2.0)
    dh_r, dE_r = OH.dense_backward(h, E, t, 0.6, n=8, c=2.0)
    np.testing.assert_allclose(obj, obj_r, rtol=2e-3, atol=2e-4)
    assert rel_l2(dh, dh_r) < 1e-2
    assert rel_l2(dE, dE_r) < 1e-2
    assert rel_l2(dh, dh_rc) < 2e-3
    assert rel_l2(dE, dE_rc) < 2e-3
    last = (V - 1) // chunk * chunk if chunk else 0
    assert rel_l2(dE[last:], dE_r[last:]) < 1e-2  # the last (ragged) chunk on its own


def test_head_streamed_rejects_bad_chunk(monkeypatch):
    from algebraic_amd.kernels import fused_head as FH
    monkeypatch.setattr(FH, "SCHEDULE", "streamed")
    monkeypatch.setattr(FH, "VOCAB_CHUNK", 300)
    h, E, t = head_inputs(128, 128, 600, seed=1, e_std=0.15)
    with pytest.raises(ValueError, match="multiple of 256"):
        run_hip(h, E, t)
