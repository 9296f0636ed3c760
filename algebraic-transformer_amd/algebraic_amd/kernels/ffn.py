"""ALU-GLU feed-forward block on MI355X with the activation fused into the products.

``alu_glu_ffn(h2, w_g, w_u, w_d, beta)`` is ``(h2 @ w_g * alu(h2 @ w_u, beta)) @ w_d`` as the
model's block computes it (src/algebraic/model.py:185-193, ffn="alu_glu"; alu and its custom VJP
src/algebraic/algebraic.py:86-113), differentiable in h2 and the three weights. The gate/up
product over the concatenated weights [w_g | w_u] carries the activation in its epilogue (one
HIP kernel writes y = gate*alu(up) and the gate/up residuals); in the backward, the product
dout @ w_d^T carries the activation's VJP in its epilogue (one HIP kernel writes
[d_gate | d_up]). The four remaining products are plain GEMMs on the same MFMA core
(``alg_ffn_gemm``), each operand read in its stored layout (no transposed copies): y @ w_d,
[d_gate | d_up] @ [w_g | w_u]^T, h2^T @ [d_gate | d_up], y^T @ dout. bf16 only; d_ff must be a
multiple of 128 and the widths multiples of 8. No CPU fallback.
"""

import torch

from .. import _lib


def _gemm(a, b, a_trans=False, b_trans=False):
    """C = op(A) op(B) in bf16 (f32 accumulation) through alg_ffn_gemm. ``a`` is stored (M, K),
    or (K, M) with ``a_trans``; ``b`` is stored (K, N), or (N, K) with ``b_trans``; both
    contiguous row-major."""
    lib = _lib.load()
    M, K = (a.shape[1], a.shape[0]) if a_trans else a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    c = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    ws_b = lib.alg_ffn_gemm_workspace_size(M, N, K)
    ws = torch.empty(max(ws_b, 1), dtype=torch.uint8, device=a.device)
    _lib.check(lib.alg_ffn_gemm(_lib.stream_of(a), M, N, K, _lib.ptr(a), a.shape[1], int(a_trans), _lib.ptr(b),
                                b.shape[1], int(b_trans), _lib.ptr(c), N, _lib.ptr(ws), ws_b), "alu_glu_ffn product")
    return c


class _FfnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h2, w_g, w_u, w_d, beta):
        lib = _lib.load()
        shape = h2.shape
        d = shape[-1]
        x = _lib.aligned16(h2).reshape(-1, d)
        N, F = x.shape[0], w_g.shape[1]
        w_gu = torch.cat([w_g, w_u], dim=1).to(torch.bfloat16).contiguous()
        wd = _lib.aligned16(w_d.to(torch.bfloat16))
        y, gate, up = (torch.empty((N, F), dtype=torch.bfloat16, device=x.device) for _ in range(3))
        _lib.check(lib.alg_ffn_alu_glu_fwd(_lib.stream_of(x), N, d, F, _lib.ptr(x), _lib.ptr(w_gu), float(beta),
                                           _lib.ptr(y), _lib.ptr(gate), _lib.ptr(up)), "alu_glu_ffn")
        out = _gemm(y, wd)
        ctx.save_for_backward(x, w_gu, wd, y, gate, up)
        ctx.meta = (shape, beta, w_g.dtype, w_u.dtype, w_d.dtype)
        return out.reshape(*shape[:-1], wd.shape[1])

    @staticmethod
    def backward(ctx, dout):
        x, w_gu, wd, y, gate, up = ctx.saved_tensors
        shape, beta, tg, tu, td = ctx.meta
        lib = _lib.load()
        N, d = x.shape
        F, dm = wd.shape
        do = _lib.aligned16(dout.to(torch.bfloat16)).reshape(N, dm)
        d_gu = torch.empty((N, 2 * F), dtype=torch.bfloat16, device=x.device)
        _lib.check(lib.alg_ffn_alu_glu_dy(_lib.stream_of(x), N, dm, F, _lib.ptr(do), _lib.ptr(wd), _lib.ptr(gate),
                                          _lib.ptr(up), float(beta), _lib.ptr(d_gu)), "alu_glu_ffn backward")
        dh2 = _gemm(d_gu, w_gu, b_trans=True).reshape(shape)
        dw_gu = _gemm(x, d_gu, a_trans=True)
        dw_d = _gemm(y, do, a_trans=True)
        return dh2, dw_gu[:, :F].to(tg), dw_gu[:, F:].to(tu), dw_d.to(td), None


def alu_glu_ffn(h2, w_g, w_u, w_d, beta: float = 0.5):
    """(h2 @ w_g * alu(h2 @ w_u, beta)) @ w_d for bfloat16 GPU tensors (model.py:185-193)."""
    if h2.dtype != torch.bfloat16:
        raise NotImplementedError(f"dtype {h2.dtype}: the gfx950 feed-forward takes bfloat16 activations")
    d = h2.shape[-1]
    if w_g.shape != w_u.shape or w_g.shape[0] != d or w_d.shape[0] != w_g.shape[1]:
        raise ValueError("w_g, w_u must be (d, d_ff) and w_d (d_ff, d_out)")
    if not h2.is_cuda:
        raise RuntimeError("alu_glu_ffn needs GPU tensors (no CPU fallback)")
    return _FfnFn.apply(h2, w_g, w_u, w_d, float(beta))
