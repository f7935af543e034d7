"""Runtime knobs honoured by the HIP engine (subset of escha_mlx/envs.py:188-326).

Read at module construction (EschaLinear / EschaMoEExperts latch them), like
the reference, so a forward never depends on call order.  Invalid values raise
ValueError naming the variable (escha_mlx/envs.py:73-82).  Boolean knobs take
the reference's spellings (escha_mlx/envs.py:89-95): surrounding blanks and
case are ignored, 1/true/yes/on and 0/false/no/off are accepted.

  ESCHA_MLX_LUT            bool table decode instead of the hash (default off)
  ESCHA_MLX_FUSED_HAD      bool Hadamard transforms fused into the GEMV / MoE
                                kernels (default on).  Off: the transforms run
                                as their own launches around the GEMV, as the
                                reference's unfused path runs them as separate
                                ops (escha_mlx/dense.py:287-298,
                                models/qwen3_5_moe.py:103-122)
  ESCHA_HIP_EXACT          bool order-exact GEMV in the modules (default off:
                                the split-K tolerance path)
  ESCHA_MLX_BLOCK_R        int  pin MoE rows per group (default: size policy)
  ESCHA_MLX_DENSE_BLOCK_R  int  pin dense rows per group (default: size policy)
  ESCHA_MLX_DENSE_MAT      bool matrix-core GEMM for dense projections of >= 16
                                rows.  Unset = on: the reference ships it off
                                (escha_mlx/msl.py:1729-1759) because the sum is
                                reassociated; on MI355X the matrix cores are the
                                prefill path, so it is on unless switched off
  ESCHA_MLX_KT_BLOCK       int  validated (1, 2, 4, 8, 16 or 32, as
                                escha_mlx/envs.py:117-121) and then unused: it
                                sets how many code tiles the reference's
                                row-blocked GEMM stages through threadgroup
                                memory per barrier pair (msl.py:1229-1242); the
                                gfx950 kernels read code straight into VGPRs and
                                stage no code tiles, so there is nothing to size

Dropped on purpose (Apple-measured negatives with no MI355X analogue, see
escha_mlx/msl.py:1145-1287): FETCH=shuffle, SPLITK, SORTX, PREFETCH,
GEMV=staged.
"""
from __future__ import annotations

import os

_TRUE = frozenset({"1", "true", "yes", "on"})
_FALSE = frozenset({"0", "false", "no", "off"})
KT_BLOCK_VALUES = (1, 2, 4, 8, 16, 32)


def parse_bool(name: str, default: bool) -> bool:
    """The boolean knob `name`: unset or empty -> default; otherwise one of the
    reference's spellings (escha_mlx/envs.py:89-95), else ValueError."""
    v = os.environ.get(name)
    if v is None or v.strip() == "":
        return default
    n = v.strip().lower()
    if n in _TRUE:
        return True
    if n in _FALSE:
        return False
    raise ValueError(f"{name} must be a boolean (0/1, false/true, no/yes, or off/on), got {v!r}")


def _int(name: str, allowed: tuple[int, ...]) -> int | None:
    v = os.environ.get(name)
    if v is None or v.strip() == "":
        return None
    try:
        n = int(v)
    except ValueError:
        raise ValueError(f"{name} must be an integer, got {v!r}") from None
    if n not in allowed:
        raise ValueError(f"{name} must be one of {allowed}, got {n}")
    return n


def use_lut() -> bool:
    return parse_bool("ESCHA_MLX_LUT", False)


def fused_had() -> bool:
    return parse_bool("ESCHA_MLX_FUSED_HAD", True)


def use_exact() -> bool:
    return parse_bool("ESCHA_HIP_EXACT", False)


def moe_one_launch() -> bool:
    """ESCHA_HIP_MOE_ONE_LAUNCH: the routed-expert path as one launch
    (esc_moe_expert_path_one_launch) wherever that launch takes the shape."""
    return parse_bool("ESCHA_HIP_MOE_ONE_LAUNCH", False)


def dense_mat() -> bool:
    return parse_bool("ESCHA_MLX_DENSE_MAT", True)


def block_r_pin() -> int | None:
    return _int("ESCHA_MLX_BLOCK_R", (1, 2, 3, 4, 8, 12, 16))


def dense_block_r_pin() -> int | None:
    return _int("ESCHA_MLX_DENSE_BLOCK_R", (1, 2, 4, 8, 16))


def kt_block() -> int:
    """ESCHA_MLX_KT_BLOCK, validated with the reference's rule (default 4);
    the value has no effect on these kernels (see the module docstring)."""
    n = _int("ESCHA_MLX_KT_BLOCK", KT_BLOCK_VALUES)
    return 4 if n is None else n
