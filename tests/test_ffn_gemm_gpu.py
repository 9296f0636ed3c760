"""GPU numerics of the feed-forward block's plain products (C ABI alg_ffn_gemm), against a
plain PyTorch float32 product of the same bf16 operands: every output element within one bf16
rounding of the f32 sum plus the f32 accumulation-order slack, bounded by the sum of |a||b|.

Covers the four stored layouts of A and B, ragged tiles in m and n, whole-tile plans, plans
whose every tile is split over k (fewer tiles than CUs), and plans that compute a first round
of whole tiles and split the rest (the 1b block's y w_d and d_gu w_gu^T shapes).
"""

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


def _run(a, b, a_trans, b_trans, M, N, K, calls=2):
    from algebraic_amd import _lib as L
    lib = L.load()
    ws_b = lib.alg_ffn_gemm_workspace_size(M, N, K)
    outs = []
    for _ in range(calls):  # a second call on a workspace holding the first call's tiles
        ws = torch.full((max(ws_b, 1),), 0x7F, dtype=torch.uint8, device="cuda")
        c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        L.check(lib.alg_ffn_gemm(L.stream_of(a), M, N, K, L.ptr(a), a.shape[1], int(a_trans), L.ptr(b), b.shape[1],
                                 int(b_trans), L.ptr(c), N, L.ptr(ws), ws_b), "alg_ffn_gemm")
        torch.cuda.synchronize()
        outs.append(c)
    return outs, ws_b


@pytest.mark.parametrize("a_trans,b_trans", LAYOUTS)
@pytest.mark.parametrize("M,N,K,split", [(296, 264, 5000, True), (264, 512, 640, False), (512, 256, 1032, False)])
def test_ffn_gemm_matches_f32(M, N, K, split, a_trans, b_trans):
    print(f"[ffn_gemm] M={M} N={N} K={K} a_trans={a_trans} b_trans={b_trans}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    B = torch.randn(K, N, device="cuda", generator=g).to(torch.bfloat16)
    a = A.t().contiguous() if a_trans else A
    b = B.t().contiguous() if b_trans else B
    outs, ws_b = _run(a, b, a_trans, b_trans, M, N, K)
    assert (ws_b > 0) == split
    ref = A.float() @ B.float()
    slack = A.float().abs() @ B.float().abs()
    for c in outs:
        err = (c.float() - ref).abs()
        tol = ref.abs() * 2.0 ** -8 + slack * 2.0 ** -20
        bad = (err > tol) | c.float().isnan()
        assert not bool(bad.any()), f"{int(bad.sum())} entries off, first {bad.nonzero()[:4].tolist()}"
    assert torch.equal(outs[0], outs[1])  # the split sum runs in a fixed order


def test_ffn_gemm_whole_round_then_split_tail():
    """272 tiles: the first 256 whole, the 16 past them split in two over k."""
    from algebraic_amd import _lib as L
    M, N, K = 4352, 4096, 2048
    assert L.load().alg_ffn_gemm_workspace_size(M, N, K) == 16 * 2 * 256 * 256 * 4
    print(f"[ffn_gemm] M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    B = torch.randn(K, N, device="cuda", generator=g).to(torch.bfloat16)
    outs, _ = _run(A, B, False, False, M, N, K, calls=1)
    ref = A.float() @ B.float()
    slack = A.float().abs() @ B.float().abs()
    err = (outs[0].float() - ref).abs()
    bad = (err > ref.abs() * 2.0 ** -8 + slack * 2.0 ** -20) | outs[0].float().isnan()
    assert not bool(bad.any()), f"{int(bad.sum())} entries off, first {bad.nonzero()[:4].tolist()}"


def test_ffn_gemm_1b_block_products():
    """The 1b block's four plain products at full size (N 16384, d 1536, d_ff 4224), in their
    stored layouts and split plans: y w_d and d_gu w_gu^T (256 whole tiles, 128 split in two),
    h2^T d_gu (198 tiles, unsplit), y^T dout (102 tiles, split five ways)."""
    N, d, F = 16384, 1536, 4224
    g = torch.Generator(device="cuda").manual_seed(11)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g).to(torch.bfloat16)
    y, wd, dgu, wgu, x, do = rn(N, F), rn(F, d), rn(N, 2 * F), rn(d, 2 * F), rn(N, d), rn(N, d)
    cases = {"y w_d": (y, wd, False, False, y, wd), "d_gu w_gu^T": (dgu, wgu, False, True, dgu, wgu.t()),
             "h2^T d_gu": (x, dgu, True, False, x.t(), dgu), "y^T dout": (y, do, True, False, y.t(), do)}
    for name, (a, b, at, bt, A, B) in cases.items():
        M, K = A.shape
        Nc = B.shape[1]
        print(f"[ffn_gemm] {name}: M={M} N={Nc} K={K}", flush=True)
        outs, _ = _run(a, b, at, bt, M, Nc, K, calls=1)
        Af, Bf = A.float(), B.float()
        ref = Af @ Bf
        tol = ref.abs() * 2.0 ** -8 + (Af.abs() @ Bf.abs()) * 2.0 ** -20
        bad = ((outs[0].float() - ref).abs() > tol) | outs[0].float().isnan()
        assert not bool(bad.any()), f"{name}: {int(bad.sum())} entries off, first {bad.nonzero()[:4].tolist()}"
        del ref, tol, bad, outs
