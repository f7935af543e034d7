"""ctypes binding of libescha_hip.so (the C ABI in include/escha_hip.h).

torch is imported first so that its bundled HIP runtime (soname
libamdhip64.so.7) is the process's runtime; the library links against the same
soname and therefore shares torch's device pointers and streams.

There is no fallback: if the library is missing or fails to load, every entry
point raises.  Build it with ``python -c "import __graft_entry__ as g; g.build()"``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime this library binds to)

LIB_NAME = "libescha_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

ESC_OK, ESC_EINVAL, ESC_EHIP, ESC_ENOSPACE, ESC_ETIMEOUT = 0, -1, -2, -3, -4

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes), exactly the declarations of include/escha_hip.h
SIGNATURES = {
    "esc_version": (_I, []),
    "esc_last_error": (ctypes.c_char_p, []),
    "esc_init": (_I, []),
    "esc_decode_tiles": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "esc_input_transform": (_I, [_P, _P, _P, _I, _I, _F, _P, _P]),
    "esc_input_transform_typed": (_I, [_P, _I, _P, _P, _I, _I, _F, _P, _P]),
    "esc_output_transform": (_I, [_P, _P, _P, _P, _I, _I, _F, _P, _P]),
    "esc_gemv": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "esc_gemv_fast_workspace": (_Z, [_I, _I, _I, _I]),
    "esc_gemv_fast_out": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _Z, _P]),
    "esc_gemm_rows": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "esc_dense_gemm_rows": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P, _P]),
    "esc_dense_gemm_rows_out": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P]),
    "esc_gemm_mfma": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "esc_gemm_mfma_out_workspace": (_Z, [_I, _I, _I, _I]),
    "esc_gemm_mfma_out": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _Z, _P]),
    "esc_linear_workspace": (_Z, [_I, _I, _I, _I]),
    "esc_linear": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _Z, _P]),
    "esc_linear_pair_workspace": (_Z, [_I, _I, _I, _I, _I, _I]),
    "esc_linear_pair": (_I, [_P, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _I, _I, _I, _F,
                             _P, _P, _P, _Z, _P]),
    "esc_linear_multi_workspace": (_Z, [_I, _I, _I, _I, _P]),
    "esc_linear_multi": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _F, _P, _P, _Z, _P]),
    "esc_gemm_rows_fast_workspace": (_Z, [_I, _I, _I, _I, _I]),
    "esc_gemm_rows_fast_out": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _Z, _P]),
    "esc_build_groups": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "esc_route_topk": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "esc_swiglu": (_I, [_P, _I, _I, _P, _P]),
    "esc_moe_combine": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "esc_w8a16": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "esc_gemv_f16w": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "esc_moe_shared_act": (_I, [_P, _P, _I, _I, _P, _P]),
    "esc_moe_block_out": (_I, [_P, _P, _P, _I, _I, _P, _P]),
    "esc_q8_embed": (_I, [_P, _I, _P, _P, _I, _I, _P, _P]),
    "esc_moe_expert_path_workspace": (_Z, [_I, _I, _I, _I, _I]),
    "esc_moe_expert_path_static_max": (_Z, []),
    "esc_decode_probe_words": (_Z, [_I, _I]),
    "esc_decode_probe": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "esc_moe_expert_path_static": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P,
                                        _P, _I, _I, _P, _P]),
    "esc_moe_status": (_I, [_P, _Z, _I, _I, _I, _I, _P, _P]),
    "esc_moe_set_spin_limit": (_I, [_I]),
    "esc_moe_layers_workspace": (_Z, [_I, _I, _I, _I, _I]),
    "esc_moe_expert_path_layers": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "esc_moe_expert_path": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P,
                                 _I, _I, _P, _P, _Z, _P]),
    "esc_moe_expert_path_one_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P,
                                            _P, _P, _I, _I, _P, _P, _Z, _P]),
}

_lib = None


class EschaHipError(RuntimeError):
    """A HIP runtime failure reported by libescha_hip."""


class EschaWaitTimeout(EschaHipError):
    """An earlier one-launch expert-path call on the device gave up a bounded
    wait between workgroups; its outputs are NaN."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is missing: the HIP engine has not been built "
            "(run __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception types."""
    if rc == ESC_OK:
        return
    msg = load().esc_last_error().decode(errors="replace")
    if rc == ESC_EINVAL:
        raise ValueError(f"{what}: {msg}")
    if rc == ESC_ENOSPACE:
        raise ValueError(f"{what}: {msg}")
    if rc == ESC_ETIMEOUT:
        raise EschaWaitTimeout(f"{what}: {msg}")
    raise EschaHipError(f"{what}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
