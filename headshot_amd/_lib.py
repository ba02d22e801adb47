"""ctypes binding of libheadshot_hip.so (the C ABI in include/headshot_hip.h).

Loading fails loudly: there is no fallback implementation. Build the
library with ``python -m headshot_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# HEADSHOT_HIP_LIB points at another build of the same library (e.g. one
# compiled with different launch-shape constants).
LIB_PATH = os.environ.get("HEADSHOT_HIP_LIB") or os.path.join(HERE, "libheadshot_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "headshot_hip.h")

HS_F32, HS_F16 = 0, 1
HS_OK, HS_EINVAL, HS_EHIP, HS_EUNSUPPORTED = 0, -1, -2, -3
ABI_VERSION = 1

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_int32  # hs_status

# name -> (restype, argtypes); mirrors include/headshot_hip.h.
SIGNATURES = {
    "hs_abi_version": (_I32, []),
    "hs_status_string": (ctypes.c_char_p, [_S]),
    "hs_last_error": (ctypes.c_char_p, []),
    "hs_layernorm": (_S, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _F]),
    "hs_gelu": (_S, [_P, _I32, _P, _P, _I64]),
    "hs_residual_ls": (_S, [_P, _I32, _P, _P, _P, _P, _I64, _I32]),
    "hs_split_heads": (_S, [_P, _I32, _P, _P, _I32, _I32, _I32, _I32]),
    "hs_rope_apply": (_S, [_P, _I32, _P, _P, _P, _I32, _I32, _I32, _I32, _I32]),
    "hs_cast_f32_to_f16": (_S, [_P, _P, _P, _I64]),
    "hs_copy_rows": (_S, [_P, _P, _I64, _P, _I64, _I64, _I64]),
    "hs_tiled_add": (_S, [_P, _P, _P, _P, _I64, _I64]),
    "hs_qknorm_rope": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F]),
    "hs_qknorm_rope_pair": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _I32, _I32, _I32, _I32, _I32, _F]),
    "hs_bias_gelu": (_S, [_P, _I32, _P, _P, _P, _I64, _I32]),
    "hs_bias_ls_residual": (_S, [_P, _I32, _P, _P, _P, _P, _P, _I64, _I32]),
    "hs_bias_ls_residual_layernorm": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32,
                                           _F]),
    "hs_assemble_tokens": (_S, [_P, _I32, _P, _I32, _P, _P, _P, _P, _P,
                                _I32, _I32, _I32, _I32, _I32]),
    "hs_linear": (_S, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32]),
    "hs_linear_gelu": (_S, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32]),
    "hs_linear_ls_residual": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32]),
    "hs_linear_qkv_heads": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _I32, _I32, _I32, _I32, _I32, _I32, _F]),
    "hs_layernorm_stats": (_S, [_P, _I32, _P, _P, _I64, _I32, _F]),
    "hs_linear_ln": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _F]),
    "hs_linear_ln_gelu": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _F]),
    "hs_linear_ln_gelu_noalloc": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _F]),
    "hs_linear_ln_qkv_heads": (_S, [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F]),
    "hs_concat_channels": (_S, [_P, _I32, _P, _P, _P, _I64, _I32, _I32]),
    "hs_cast_f16_to_f32": (_S, [_P, _P, _P, _I64]),
    "hs_cache_build": (_S, [_P, _I32, _P, _P, _P, _I64, _I32, _I32]),
    "hs_copy_row_blocks": (_S, [_P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64]),
    "hs_attention": (_S, [_P, _I32, _P, _P, _P, _P, _I32, _I32, _I32, _I32]),
    "hs_attn_merge": (_S, [_P, _I32, _P, _P, _I32, _I32, _I32, _I32]),
    "hs_attention_merged": (_S, [_P, _I32, _P, _P, _P, _P, _I32, _I32, _I32, _I32]),
    "hs_rope_periods": (None, [_P]),
    "hs_rope_tables": (_S, [_P, _I32, _I32, _P, _P]),
}


class HsError(RuntimeError):
    """A failing status from the library (HS_EHIP / HS_EUNSUPPORTED)."""

    def __init__(self, status: int, op: str, message: str):
        super().__init__(f"{op}: {message} ({status_name(status)})")
        self.status = status


class HsContractError(HsError, AssertionError):
    """HS_EINVAL: a contract violation (the reference panics on these)."""


_lib = None


def header_functions(path: str = HEADER) -> list[str]:
    """Names of the functions include/headshot_hip.h declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"libheadshot_hip.so not found at {path}; build it with "
            "`python -m headshot_amd.build` (there is no fallback path)")
    # PyTorch ships its own HIP runtime under the same soname
    # (libamdhip64.so.7). Whichever copy is loaded first serves the whole
    # process, and stream handles from one runtime instance are meaningless
    # to another, so torch's copy must be in place before this library
    # resolves its dependency.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    got = lib.hs_abi_version()
    if got != ABI_VERSION:
        raise ImportError(f"libheadshot_hip ABI {got}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def status_name(status: int) -> str:
    return {HS_OK: "HS_OK", HS_EINVAL: "HS_EINVAL", HS_EHIP: "HS_EHIP",
            HS_EUNSUPPORTED: "HS_EUNSUPPORTED"}.get(status, f"status {status}")


def check(status: int, op: str) -> None:
    if status == HS_OK:
        return
    msg = (load().hs_last_error() or b"").decode(errors="replace")
    if status == HS_EINVAL:
        raise HsContractError(status, op, msg)
    raise HsError(status, op, msg)
