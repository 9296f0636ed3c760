"""CPU: the C ABI library loads and exports every symbol include/algebraic_hip.h declares.

No compute calls are made (no GPU here); the host-side validation that runs before any
launch is exercised through calls whose arguments fail validation.
"""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "algebraic_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(alg_[a-z0-9_]+)\s*\(", text)))


def lib():
    from algebraic_amd import _lib
    try:
        return _lib.load()
    except _lib.HipLibraryMissing as e:  # built by __graft_entry__.build()
        pytest.fail(str(e))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("alg_attn_prepare", "alg_attn_fwd", "alg_attn_bwd", "alg_head_fwd", "alg_head_bwd",
              "alg_attn_workspace_size", "alg_head_workspace_size", "alg_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    handle = lib()
    for name in declared_functions():
        assert hasattr(handle, name), name
    from algebraic_amd import _lib
    assert set(declared_functions()) == set(_lib.EXPORTS)


def test_abi_version_matches_the_header():
    """The library reports the ALG_ABI_VERSION of the header it was built from, and the
    Python bindings (whose signatures follow that header) expect the same version."""
    from algebraic_amd import _lib
    m = re.search(r"#define\s+ALG_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert m, "ALG_ABI_VERSION missing from the header"
    assert lib().alg_abi_version() == int(m.group(1)) == _lib.ABI_VERSION
    assert f"ABI {_lib.ABI_VERSION}" in lib().alg_version().decode()


def test_workspace_sizes():
    from algebraic_amd import _lib
    handle = lib()
    B, H, T, D = 8, 16, 2048, 128
    ws32 = handle.alg_attn_workspace_size(_lib.DTYPE_F32, B, H, T, D)
    ws16 = handle.alg_attn_workspace_size(_lib.DTYPE_BF16, B, H, T, D)
    assert ws32 >= B * H * T * D * 4           # f32 dQ accumulator
    assert 0 < ws16 < 1 << 20                  # bf16: the sink and guard partials only
    assert handle.alg_attn_workspace_size(_lib.DTYPE_BF16, 0, H, T, D) == 0
    assert handle.alg_attn_workspace_size(7, B, H, T, D) == 0
    bf, f32 = _lib.DTYPE_BF16, _lib.DTYPE_F32
    fwd = handle.alg_head_workspace_size(bf, 16384, 2048, 32000, 0)
    bwd = handle.alg_head_workspace_size(bf, 16384, 2048, 32000, 1)
    assert bwd - fwd >= 32000 * 16384 * 2     # bf16 logit-gradient block (recompute schedule)
    bwd_res = handle.alg_head_workspace_size(bf, 16384, 2048, 32000, 2)
    assert bwd_res - fwd >= 16384 * 2048 * 2  # bf16 s*h/l (residual schedule)
    assert handle.alg_head_residual_size(16384, 2048, 32000) >= 32000 * 16384 * 2 + 16384 * 4
    # f32 hidden states: the f32 logit-gradient block, no residual schedule.
    fwd32 = handle.alg_head_workspace_size(f32, 16384, 2048, 32000, 0)
    bwd32 = handle.alg_head_workspace_size(f32, 16384, 2048, 32000, 1)
    assert fwd32 > 0 and bwd32 - fwd32 >= 32000 * 16384 * 4
    assert handle.alg_head_workspace_size(f32, 16384, 2048, 32000, 2) == 0
    assert handle.alg_head_workspace_size(f32, 512, 256, 1000, 3) > 0
    assert handle.alg_head_workspace_size(7, 512, 256, 1000, 0) == 0
    # Streamed backward at C4b: the default chunk is 8192 vocabulary rows (32 x 8 = 256 dE
    # tiles), so the workspace holds one 16384 x 8192 bf16 block and the f32 dh accumulator,
    # no (N, V) block.
    sw = handle.alg_head_streamed_workspace_size(bf, 16384, 2048, 32000, 0)
    assert sw == 16384 * 8192 * 2 + 16384 * 2048 * 4
    assert sw < 0.4 * (bwd - fwd)
    # 4096-row chunks: the last chunk (3328 rows, 104 dE tiles) splits its dE tiles over 7
    # token ranges, whose f32 tiles the workspace holds as well.
    assert (handle.alg_head_streamed_workspace_size(bf, 16384, 2048, 32000, 4096)
            == 16384 * 4096 * 2 + 16384 * 2048 * 4 + 104 * 7 * 256 * 256 * 4)
    assert handle.alg_head_streamed_workspace_size(bf, 16384, 2048, 32000, 32768) == 16384 * 32000 * 2  # one chunk
    assert handle.alg_head_streamed_workspace_size(f32, 16384, 2048, 32000, 4096) == 16384 * 4096 * 4
    assert handle.alg_head_streamed_workspace_size(bf, 16384, 2048, 32000, 300) == 0   # not a multiple of 256
    assert handle.alg_head_streamed_workspace_size(bf, 16384, 2048, 32000, -256) == 0
    assert handle.alg_head_streamed_workspace_size(7, 16384, 2048, 32000, 0) == 0


def test_invalid_arguments_fail_before_launch():
    from algebraic_amd import _lib
    handle = lib()
    P = ctypes.c_void_p
    # D = 96 is not built; no pointer is touched before validation.
    rc = handle.alg_attn_fwd(None, 0, 0, 1, 1, 64, 96, P(16), P(16), P(16), None, 16, 3, P(16), 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED
    assert b"head_dim" in handle.alg_last_error()
    rc = handle.alg_attn_fwd(None, 0, 0, 1, 1, 64, 64, P(16), P(16), P(16), None, 12, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"power of two" in handle.alg_last_error()
    # Any power of two up to 2^20 (the reference takes any power of two, flash.py:740-741).
    rc = handle.alg_attn_fwd(None, 0, 0, 1, 1, 64, 64, P(16), P(16), P(16), None, 1 << 21, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"2^20" in handle.alg_last_error()
    rc = handle.alg_head_fwd(None, 0, 128, 256, 1000, P(16), P(16), P(16), 3, 2.0, P(16), P(16), P(16), P(16),
                             None, P(16), 1 << 30)
    assert rc == _lib.ALG_ERR_INVALID and b"power of two" in handle.alg_last_error()
    rc = handle.alg_attn_fwd(None, 0, 2, 1, 1, 64, 64, P(16), P(16), P(16), None, 16, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"layout" in handle.alg_last_error()
    # (B, T, H, D): one head's rows must stay within 32-bit byte offsets.
    rc = handle.alg_attn_fwd(None, 0, 1, 1, 256, 1 << 16, 128, P(16), P(16), P(16), None, 16, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"layout" in handle.alg_last_error()
    rc = handle.alg_head_fwd(None, 0, 128, 100, 1000, P(16), P(16), P(16), 8, 2.0, P(16), P(16), P(16), P(16),
                             None, P(16), 1 << 30)  # d = 100: rows not 16-byte aligned
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"d_model" in handle.alg_last_error()
    rc = handle.alg_head_bwd(None, 0, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 8, 2.0, None, P(16),
                             P(16), 0, P(16), 16)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()
    rc = handle.alg_head_bwd_streamed(None, 0, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 8, 2.0, 300,
                                      P(16), P(16), 0, P(16), 1 << 30)
    assert rc == _lib.ALG_ERR_INVALID and b"vocab_chunk" in handle.alg_last_error()
    rc = handle.alg_head_bwd_streamed(None, 0, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 1, 2.0, 256,
                                      P(16), P(16), 0, P(16), 16)  # n = 1 is fine: no residual
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()
    # n = 1 (fused_head.py:269-272 accepts it): with a residual it is refused (that schedule
    # needs stat^n = 1/l, which the reference's l^(-1/n) = rsqrt(l) at n = 1 does not give);
    # without one it passes the n check and fails here only on the too-small workspace.
    rc = handle.alg_head_fwd(None, 0, 128, 256, 1000, P(16), P(16), P(16), 1, 2.0, P(16), P(16), P(16), P(16),
                             P(16), P(16), 16)
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"n = 1" in handle.alg_last_error()
    rc = handle.alg_head_fwd(None, 0, 128, 256, 1000, P(16), P(16), P(16), 1, 2.0, P(16), P(16), P(16), P(16),
                             None, P(16), 16)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()
    # f32 hidden states take no residual; an unknown dtype is refused.
    rc = handle.alg_head_fwd(None, _lib.DTYPE_F32, 128, 256, 1000, P(16), P(16), P(16), 8, 2.0, P(16), P(16),
                             P(16), P(16), P(16), P(16), 1 << 30)
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"residual" in handle.alg_last_error()
    rc = handle.alg_head_bwd(None, 5, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 8, 2.0, None, P(16),
                             P(16), 0, P(16), 1 << 30)
    assert rc == _lib.ALG_ERR_INVALID and b"dtype" in handle.alg_last_error()
    rc = handle.alg_head_bwd(None, _lib.DTYPE_F32, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 8, 2.0, None,
                             P(16), P(16), 1, P(16), 16)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.ALG_ERR_INVALID, "probe")


def test_guarded_forward_validates_before_launch():
    """alg_attn_fwd_guarded: the guard applies for n <= 32 (flash.py:834); the workspace holds
    one set of guard maxima per 128-query workgroup; argument errors precede any launch."""
    from algebraic_amd import _lib
    handle = lib()
    P = ctypes.c_void_p
    bf = _lib.DTYPE_BF16
    B, H, T, D = 2, 4, 3000, 128
    ws = handle.alg_attn_workspace_size(bf, B, H, T, D)
    assert ws >= 3 * 4 * B * H * ((T + 127) // 128)

    def call(n=16, c=8.0, nsink=4, sink=P(16), q=P(16), ws_bytes=ws):
        return handle.alg_attn_fwd_guarded(None, bf, 0, B, H, T, D, q, P(16), P(16), sink, nsink, c, n, P(16),
                                           P(16), P(16), P(16), None, P(16), P(16), ws_bytes)

    assert call(n=64) == _lib.ALG_ERR_INVALID and b"n <= 32" in handle.alg_last_error()
    assert call(n=12) == _lib.ALG_ERR_INVALID and b"power of two" in handle.alg_last_error()
    assert call(c=0.0) == _lib.ALG_ERR_INVALID and b"positive" in handle.alg_last_error()
    assert call(nsink=3) == _lib.ALG_ERR_INVALID and b"sink_count" in handle.alg_last_error()
    assert call(q=None) == _lib.ALG_ERR_INVALID and b"required" in handle.alg_last_error()
    assert call(q=P(18)) == _lib.ALG_ERR_INVALID and b"aligned" in handle.alg_last_error()
    assert call(ws_bytes=ws - 1) == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()


def test_neighbour_entry_points_validate_before_launch():
    """The prologue, eval head, final norm and feed-forward entry points reject bad shapes,
    missing workspaces, non-finite scalars and misaligned matrices before any launch."""
    from algebraic_amd import _lib
    handle = lib()
    P = ctypes.c_void_p
    err = lambda: handle.alg_last_error()
    # Fused prologue: cos without sin, bad eps, workspace too small.
    args = [None, 0, 1, 2, 4, 128, 128, P(16), P(16), P(16), None, None, P(16), None, 1e-5, None, 0, 8.0, 16, 1,
            P(16), P(16), P(16), P(16), None, P(16), P(16), 1 << 30]
    rc = handle.alg_attn_qk_prologue(*args)
    assert rc == _lib.ALG_ERR_INVALID and b"cos and sin" in err()
    args[12] = None
    args[14] = 0.0
    rc = handle.alg_attn_qk_prologue(*args)
    assert rc == _lib.ALG_ERR_INVALID and b"eps" in err()
    args[14] = 1e-5
    args[-1] = 16
    rc = handle.alg_attn_qk_prologue(*args)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in err()
    assert handle.alg_attn_prologue_workspace_size(2, 4, 128, 128) > 16
    rc = handle.alg_cayley_tables(None, P(16), 0, 128, P(16), P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"positive" in err()
    # Eval head: pass 3 sizes its workspace; too small is refused.
    for dt in (_lib.DTYPE_BF16, _lib.DTYPE_F32):
        need = handle.alg_head_workspace_size(dt, 512, 256, 1000, 3)
        assert need > 0
        rc = handle.alg_head_eval(None, dt, 512, 256, 1000, P(16), P(16), P(16), 8, 2.0, P(16), P(16), P(16),
                                  need - 1)
        assert rc == _lib.ALG_ERR_INVALID and b"workspace" in err()
    # Final norm: width limits, eps, gain gradient without a gain, alignment.
    rc = handle.alg_rms_norm_fwd(None, 4, 100, P(16), None, 1e-5, P(16), P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"16-byte" in err()
    rc = handle.alg_rms_norm_fwd(None, 4, 8192, P(16), None, 1e-5, P(16), P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"at most" in err()
    rc = handle.alg_rms_norm_fwd(None, 4, 256, P(16), None, float("nan"), P(16), P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"eps" in err()
    rc = handle.alg_rms_norm_fwd(None, 4, 256, P(18), None, 1e-5, P(16), P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in err()
    rc = handle.alg_rms_norm_bwd(None, 4, 256, P(16), None, P(16), P(16), P(16), P(16), P(16), 1 << 20)
    assert rc == _lib.ALG_ERR_INVALID and b"gain" in err()
    rc = handle.alg_rms_norm_bwd(None, 4, 256, P(16), P(16), P(16), P(16), P(16), P(16), P(16), 4)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in err()
    assert handle.alg_rms_norm_workspace_size(16384, 2048) >= 2048 * 4
    # Feed-forward: d_ff % 128, non-finite beta, misaligned matrices.
    rc = handle.alg_ffn_alu_glu_fwd(None, 256, 128, 200, P(16), P(16), 0.5, P(16), P(16), P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"128" in err()
    rc = handle.alg_ffn_alu_glu_fwd(None, 256, 128, 256, P(16), P(16), float("inf"), P(16), P(16), P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"beta" in err()
    rc = handle.alg_ffn_alu_glu_fwd(None, 256, 128, 256, P(16), P(16), 0.5, P(16), P(24), P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in err()
    rc = handle.alg_ffn_alu_glu_dy(None, 256, 128, 256, P(16), P(16), P(16), P(16), 0.5, P(20))
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in err()
    # Plain feed-forward products: row lengths and leading dimensions, workspace of a split plan.
    rc = handle.alg_ffn_gemm(None, 256, 100, 512, P(16), 512, 0, P(16), 104, 0, P(16), 104, None, 0)
    assert rc == _lib.ALG_ERR_INVALID and b"multiples of 8" in err()
    rc = handle.alg_ffn_gemm(None, 300, 256, 512, P(16), 512, 1, P(16), 256, 0, P(16), 256, None, 0)
    assert rc == _lib.ALG_ERR_INVALID and b"multiples of 8" in err()  # A stored (K, M): M = 300
    rc = handle.alg_ffn_gemm(None, 256, 256, 512, P(16), 256, 0, P(16), 256, 0, P(16), 256, None, 0)
    assert rc == _lib.ALG_ERR_INVALID and b"leading" in err()  # lda < K
    rc = handle.alg_ffn_gemm(None, 256, 256, 512, P(16), 512, 0, P(24), 256, 0, P(16), 256, None, 0)
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in err()
    assert handle.alg_ffn_gemm_workspace_size(256, 256, 512) == 0       # one tile, short k: no split
    need = handle.alg_ffn_gemm_workspace_size(296, 264, 5000)           # 4 tiles, k split 4 ways
    assert need == 4 * 4 * 256 * 256 * 4
    rc = handle.alg_ffn_gemm(None, 296, 264, 5000, P(16), 5000, 0, P(16), 264, 0, P(16), 264, P(16), need - 1)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in err()
    # The 1b block's products: y w_d and d_gu w_gu^T split their last 128 of 384 tiles in two,
    # h2^T d_gu (198 tiles) is not split, y^T dout (102 tiles) is split five ways.
    assert handle.alg_ffn_gemm_workspace_size(16384, 1536, 4224) == 128 * 2 * 256 * 256 * 4
    assert handle.alg_ffn_gemm_workspace_size(16384, 1536, 8448) == 128 * 2 * 256 * 256 * 4
    assert handle.alg_ffn_gemm_workspace_size(1536, 8448, 16384) == 0
    assert handle.alg_ffn_gemm_workspace_size(4224, 1536, 16384) == 102 * 5 * 256 * 256 * 4


def test_noalloc_backward_rejects_scratch_beyond_its_limit():
    """alg_attn_bwd_noalloc refuses, before any launch or device call, a shape whose scratch
    (here an f32 dQ accumulator of 2 x 12 x 1024 x 128 floats) exceeds the per-GPU array."""
    from algebraic_amd import _lib
    handle = lib()
    P = ctypes.c_void_p
    B, H, T, D = 2, 12, 1024, 128
    assert handle.alg_attn_workspace_size(_lib.DTYPE_F32, B, H, T, D) > 8 << 20
    rc = handle.alg_attn_bwd_noalloc(None, _lib.DTYPE_F32, 0, B, H, T, D, P(16), P(16), P(16), None, P(16), P(16),
                                     P(16), 16, 3, P(16), 60.0, 1, 1, 0.01, P(16), P(16), P(16), P(16), None)
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"scratch" in handle.alg_last_error()
    rc = handle.alg_attn_bwd_noalloc(None, _lib.DTYPE_BF16, 0, B, H, T, 96, P(16), P(16), P(16), None, P(16),
                                     P(16), P(16), 16, 3, P(16), 60.0, 1, 1, 0.01, P(16), P(16), P(16), P(16), None)
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"head_dim" in handle.alg_last_error()


def test_hot_path_entry_points_reject_misaligned_matrices():
    """Attention and head matrices are moved 16 bytes per lane: a base off a 16-byte boundary
    is refused before any launch."""
    from algebraic_amd import _lib
    handle = lib()
    P = ctypes.c_void_p
    rc = handle.alg_attn_fwd(None, 0, 0, 1, 1, 64, 64, P(18), P(16), P(16), None, 16, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in handle.alg_last_error()
    rc = handle.alg_head_fwd(None, 0, 128, 256, 1000, P(16), P(40), P(16), 8, 2.0, P(16), P(16), P(16), P(16),
                             None, P(16), 1 << 30)
    assert rc == _lib.ALG_ERR_INVALID and b"aligned" in handle.alg_last_error()


def test_sources_stay_capture_safe():
    """The entry points must stay safe under stream capture (tests/test_graph_gpu.py replays the
    whole step from one graph): no device allocation, no memset or copy (a memset recorded
    into a graph is a hazard of its own), no host synchronisation in the library's sources.
    The one exception is the opt-in kernel timer's report, which the host calls outside any
    step (alg_timer_report)."""
    banned = re.compile(r"\b(hipMalloc\w*|hipFree\w*|hipMemset\w*|hipMemcpy\w*|hipDeviceSynchronize|"
                        r"hipStreamSynchronize|hipStreamQuery|hipEventQuery|hipHostMalloc|hipExtMallocWithFlags)\s*\(")
    found = []
    for path in sorted((ROOT / "algebraic-transformer_amd" / "csrc").glob("*")):
        if path.suffix not in (".hip", ".h", ".cpp"):
            continue
        for i, line in enumerate(path.read_text().splitlines(), 1):
            code = line.split("//", 1)[0]
            if banned.search(code):
                found.append(f"{path.name}:{i}: {line.strip()}")
    assert not found, found
    timer = (ROOT / "algebraic-transformer_amd" / "csrc" / "ktimer.hip").read_text()
    assert timer.count("hipEventSynchronize(") == 1, "the timer report is the only synchronising call"
