"""CPU: the host mirror raises the reference's errors before touching a GPU.

Mirrors the ValueErrors of src/algebraic/kernels/flash.py:740-743, 796-797, 802-817, 836 and
src/algebraic/kernels/fused_head.py:163-164, 269-272, plus NotImplementedError for the
softmax / cross-entropy control arms that this build does not provide.
"""

import pytest

torch = pytest.importorskip("torch")

from algebraic_amd.kernels.flash import flash_attention, make_variant  # noqa: E402
from algebraic_amd.kernels.fused_head import fused_head  # noqa: E402


def qkv(T=256, D=64, dtype=torch.bfloat16):
    return [torch.zeros(1, 2, T, D, dtype=dtype) for _ in range(3)]


def test_make_variant_matches_reference_defaults():
    v = make_variant("asinh", 16, 8.0, 2048)
    assert not v.shift and v.fast_rho and v.inv_stat and abs(v.clamp - 63.7) < 0.05
    assert make_variant("asinh", 16, 8.0, 10 ** 30).shift  # clamp < 20 -> shifted
    with pytest.raises(ValueError):
        make_variant("asinh", 12, 8.0)
    with pytest.raises(ValueError):
        make_variant("asinh", 16, -1.0)
    with pytest.raises(ValueError):
        make_variant("asinh", 16, 8.0, inv_stat=True, shift=True)
    with pytest.raises(ValueError):
        make_variant("nope")


def test_flash_validation():
    q, k, v = qkv(T=256)
    with pytest.raises(ValueError):
        flash_attention(q, k, v, kind="asinh", block=96)          # 256 % 96
    with pytest.raises(ValueError):
        flash_attention(q, k, v, kind="asinh", n=6)
    with pytest.raises(ValueError):
        flash_attention(q, k, v, kind="asinh", resident_bwd=True)  # needs T in {512,1024,2048}
    with pytest.raises(ValueError):
        flash_attention(q, k, v, kind="asinh", poly_rho=True, range_guard=True)
    # test_whole_head_residency_rejects_unsupported_shape (test_flash_kernel_tpu.py:337-341).
    x = torch.ones((1, 1, 512, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="whole-head residency"):
        flash_attention(x, x, x, kind="asinh", c=8.0, head_resident=True)
    with pytest.raises(NotImplementedError):
        flash_attention(q, k, v, kind="softmax")
    q16, k16, v16 = qkv(dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        flash_attention(q16, k16, v16, kind="asinh", range_guard=True)
    with pytest.raises(RuntimeError):
        flash_attention(q, k, v, kind="asinh", range_guard=True)   # CPU tensors: no fallback
    # Widths other than the built 64 / 128 run zero-padded up to 128 (GPU only); above 128 the
    # call is refused before any device work.
    x = torch.ones((1, 1, 64, 160), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="head_dim 160"):
        flash_attention(x, x, x, kind="asinh", range_guard=True)
    x = torch.ones((1, 1, 64, 96), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_attention(x, x, x, kind="asinh", range_guard=True)


def test_fused_head_validation():
    h = torch.zeros(256, 128, dtype=torch.bfloat16)
    E = torch.zeros(300, 128)
    t = torch.zeros(256, dtype=torch.int32)
    with pytest.raises(ValueError):
        fused_head(h, E, t, kind="xent")
    with pytest.raises(ValueError):
        fused_head(h, E, t, kind="alg_ce", n=6)
    with pytest.raises(ValueError):
        fused_head(h[:200], E, t[:200], kind="alg_ce", block_n=128)   # 200 % 128
    with pytest.raises(NotImplementedError):
        fused_head(h, E, t, kind="ce")
    with pytest.raises(NotImplementedError):
        fused_head(h.half(), E, t, kind="alg_ce")                    # bf16 or f32 hidden states only
    with pytest.raises(RuntimeError):
        fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)               # CPU tensors: no fallback
    with pytest.raises(RuntimeError):
        fused_head(h.float(), E, t, kind="alg_ce", n=8, c=2.0)


def test_neighbour_mirrors_validate_before_any_launch():
    """The final norm, feed-forward, eval head and prologue mirrors refuse unsupported dtypes,
    CPU tensors (no host fallback) and inconsistent shapes before touching a GPU."""
    from algebraic_amd.kernels.ffn import alu_glu_ffn
    from algebraic_amd.kernels.fused_head import head_logprob
    from algebraic_amd.kernels.norm import rms_norm
    from algebraic_amd.kernels.prologue import cayley_powers, cayley_table_geometric
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        rms_norm(x.float())
    with pytest.raises(RuntimeError):
        rms_norm(x)
    with pytest.raises(ValueError):
        rms_norm(x, torch.ones(128))
    h2, wg, wd = torch.zeros(8, 64, dtype=torch.bfloat16), torch.zeros(64, 128), torch.zeros(128, 64)
    with pytest.raises(NotImplementedError):
        alu_glu_ffn(h2.float(), wg, wg, wd)
    with pytest.raises(ValueError):
        alu_glu_ffn(h2, wg, wg[:, :64], wd)
    with pytest.raises(RuntimeError):
        alu_glu_ffn(h2, wg, wg, wd)
    h, E, t = torch.zeros(16, 64, dtype=torch.bfloat16), torch.zeros(100, 64), torch.zeros(16, dtype=torch.int32)
    # n = 1 passes the reference's power-of-two check (fused_head.py:269-272) and is taken
    # (the recompute schedule); on CPU tensors it stops at the device check like any n.
    from algebraic_amd.kernels.fused_head import fused_head
    with pytest.raises(RuntimeError, match="GPU"):
        fused_head(h, E, t, kind="alg_ce", n=1, c=2.0)
    with pytest.raises(NotImplementedError):
        head_logprob(h, E, t, head="ce")
    with pytest.raises(ValueError):
        head_logprob(h, E, t, n=6)
    with pytest.raises(NotImplementedError):
        head_logprob(h.half(), E, t)
    with pytest.raises(RuntimeError):
        head_logprob(h, E, t)
    with pytest.raises(RuntimeError):
        head_logprob(h.float(), E, t)
    with pytest.raises(ValueError):
        cayley_table_geometric(96, 128)           # head_dim / 2 = 48: not a power of two
    with pytest.raises(ValueError):
        cayley_powers(torch.zeros(2, 4), 8)
    with pytest.raises(RuntimeError):
        cayley_powers(torch.zeros(4), 8)
