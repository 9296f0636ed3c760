"""ctypes binding of libalgebraic_hip.so (the C ABI declared in include/algebraic_hip.h).

The library is the product path: if it is missing, or a call is made without a GPU, the
functions here raise. There is no CPU fallback.
"""

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("ALGEBRAIC_HIP_LIB", _HERE / "libalgebraic_hip.so"))

ABI_VERSION = 2  # ALG_ABI_VERSION of include/algebraic_hip.h these signatures follow

ALG_OK, ALG_ERR_INVALID, ALG_ERR_UNSUPPORTED, ALG_ERR_HIP = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F32 = 0, 1
ATTN_INRANGE, ATTN_CLIPPED, ATTN_SHIFTED, ATTN_GUARDED = 0, 1, 2, 3
LAYOUT_BHTD, LAYOUT_BTHD = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t
_L = ctypes.c_long

_SIGNATURES = {
    "alg_last_error": (ctypes.c_char_p, []),
    "alg_version": (ctypes.c_char_p, []),
    "alg_abi_version": (_I, []),
    "alg_attn_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "alg_attn_prepare": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _F, _I, _I, _P, _P, _P, _P, _S]),
    "alg_attn_fwd": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P, _F, _I, _I, _P, _P, _P]),
    "alg_attn_fwd_guarded": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _F, _I, _P, _P, _P, _P, _P, _P,
                                  _P, _S]),
    "alg_attn_bwd": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _F, _I, _I, _F,
                          _P, _P, _P, _P, _P, _P, _S]),
    "alg_attn_bwd_noalloc": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _F, _I, _I,
                                  _F, _P, _P, _P, _P, _P]),
    "alg_attn_prologue_workspace_size": (_S, [_I, _I, _I, _I]),
    "alg_cayley_tables": (_I, [_P, _P, _I, _I, _P, _P]),
    "alg_attn_qk_prologue": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _F, _P, _I, _F, _I, _I,
                                  _P, _P, _P, _P, _P, _P, _P, _S]),
    "alg_attn_qk_prologue_bwd": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _P, _P, _P, _S]),
    "alg_head_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "alg_head_residual_size": (_S, [_I, _I, _I]),
    "alg_head_fwd": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _I, _F, _P, _P, _P, _P, _P, _P, _S]),
    "alg_head_bwd": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _F, _P, _P, _P, _I, _P, _S]),
    "alg_head_streamed_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "alg_head_bwd_streamed": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _F, _I, _P, _P, _I, _P, _S]),
    "alg_head_eval": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _I, _F, _P, _P, _P, _S]),
    "alg_rms_norm_workspace_size": (_S, [_I, _I]),
    "alg_ffn_alu_glu_fwd": (_I, [_P, _I, _I, _I, _P, _P, _F, _P, _P, _P]),
    "alg_ffn_alu_glu_dy": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _F, _P]),
    "alg_ffn_gemm_workspace_size": (_S, [_I, _I, _I]),
    "alg_ffn_gemm": (_I, [_P, _I, _I, _I, _P, _L, _I, _P, _L, _I, _P, _L, _P, _S]),
    "alg_rms_norm_fwd": (_I, [_P, _I, _I, _P, _P, _F, _P, _P]),
    "alg_rms_norm_bwd": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _S]),
    "alg_timer_enable": (None, [_I]),
    "alg_timer_report": (_S, [ctypes.c_char_p, _S]),
}

EXPORTS = tuple(_SIGNATURES)

_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def load():
    """Load the shared library once; raise HipLibraryMissing if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipLibraryMissing(
            f"{LIB_PATH} not found: build it with `python algebraic-transformer_amd/build_lib.py` "
            "(or __graft_entry__.build()); the algebraic kernels have no CPU fallback")
    lib = ctypes.CDLL(str(LIB_PATH))
    if not hasattr(lib, "alg_abi_version"):
        raise HipLibraryMissing(f"{LIB_PATH} predates ABI version {ABI_VERSION}: rebuild it")
    lib.alg_abi_version.restype = ctypes.c_int
    lib.alg_abi_version.argtypes = []
    if lib.alg_abi_version() != ABI_VERSION:
        raise HipLibraryMissing(f"{LIB_PATH} has ABI version {lib.alg_abi_version()}, these bindings "
                                f"expect {ABI_VERSION}: rebuild it")
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what):
    """Raise the Python error matching a C ABI status code."""
    if rc == ALG_OK:
        return
    msg = load().alg_last_error().decode(errors="replace")
    if rc == ALG_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == ALG_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def timer_enable(on=True):
    """Record a HIP event pair around every kernel launch of the library (measurement)."""
    load().alg_timer_enable(1 if on else 0)


def timer_report():
    """Per-kernel {name: {"launches", "mean_ms"}} since the last report (synchronises)."""
    import json
    buf = ctypes.create_string_buffer(1 << 20)
    n = load().alg_timer_report(buf, len(buf))
    if n > len(buf):
        raise RuntimeError("timer report truncated")
    return json.loads(buf.value.decode())


def aligned16(t):
    """``t`` contiguous and starting on a 16-byte boundary (copied if needed), as the kernels
    that move 8 bf16 per lane require."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def ptr(t):
    """Device pointer of a tensor (or None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
