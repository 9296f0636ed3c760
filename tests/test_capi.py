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


def test_workspace_sizes():
    handle = lib()
    B, H, T, D = 8, 16, 2048, 128
    ws = handle.alg_attn_workspace_size(B, H, T, D)
    assert ws >= B * H * T * D * 4           # f32 dQ accumulator
    assert handle.alg_attn_workspace_size(0, H, T, D) == 0
    fwd = handle.alg_head_workspace_size(16384, 2048, 32000, 0)
    bwd = handle.alg_head_workspace_size(16384, 2048, 32000, 1)
    assert bwd - fwd >= 32000 * 16384 * 2     # bf16 logit-gradient block (recompute schedule)
    bwd_res = handle.alg_head_workspace_size(16384, 2048, 32000, 2)
    assert bwd_res - fwd >= 16384 * 2048 * 2  # bf16 s*h/l (residual schedule)
    assert handle.alg_head_residual_size(16384, 2048, 32000) >= 32000 * 16384 * 2 + 16384 * 4


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
    rc = handle.alg_attn_fwd(None, 0, 2, 1, 1, 64, 64, P(16), P(16), P(16), None, 16, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_INVALID and b"layout" in handle.alg_last_error()
    # (B, T, H, D): one head's rows must stay within 32-bit byte offsets.
    rc = handle.alg_attn_fwd(None, 0, 1, 1, 256, 1 << 16, 128, P(16), P(16), P(16), None, 16, 0, None, 0.0, 1, 1,
                             P(16), None, P(16))
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"layout" in handle.alg_last_error()
    rc = handle.alg_head_fwd(None, 128, 100, 1000, P(16), P(16), P(16), 8, 2.0, P(16), P(16), P(16), P(16),
                             None, P(16), 1 << 30)  # d = 100: rows not 16-byte aligned
    assert rc == _lib.ALG_ERR_UNSUPPORTED and b"d_model" in handle.alg_last_error()
    rc = handle.alg_head_bwd(None, 128, 256, 1000, P(16), P(16), P(16), P(16), P(16), 8, 2.0, None, P(16), P(16),
                             0, P(16), 16)
    assert rc == _lib.ALG_ERR_INVALID and b"workspace" in handle.alg_last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.ALG_ERR_INVALID, "probe")
