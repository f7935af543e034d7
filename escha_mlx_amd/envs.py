"""Runtime knobs honoured by the HIP engine (subset of escha_mlx/envs.py:188-326).

Read at module construction (EschaLinear / EschaMoEExperts latch them), like
the reference, so a forward never depends on call order.  Invalid values raise
ValueError naming the variable (escha_mlx/envs.py:73-82).

  ESCHA_MLX_LUT            0/1  table decode instead of the hash (default 0)
  ESCHA_HIP_EXACT          0/1  order-exact GEMV in the modules (default 0:
                                the split-K tolerance path)
  ESCHA_MLX_BLOCK_R        int  pin MoE rows per group (default: size policy)
  ESCHA_MLX_DENSE_BLOCK_R  int  pin dense rows per group (default: size policy)
  ESCHA_MLX_DENSE_MAT      0/1  matrix-core GEMM for dense projections of >= 16
                                rows.  Unset = on: the reference ships it off
                                (escha_mlx/msl.py:1729-1759) because the sum is
                                reassociated; on MI355X the matrix cores are the
                                prefill path, so it is on unless set to 0

Dropped on purpose (Apple-measured negatives with no MI355X analogue, see
escha_mlx/msl.py:1145-1287): FETCH=shuffle, SPLITK, SORTX, PREFETCH,
GEMV=staged.
"""
from __future__ import annotations

import os


def _flag(name: str, default: bool) -> bool:
    v = os.environ.get(name)
    if v is None or v == "":
        return default
    if v not in ("0", "1"):
        raise ValueError(f"{name} must be 0 or 1, got {v!r}")
    return v == "1"


def _int(name: str, allowed: tuple[int, ...]) -> int | None:
    v = os.environ.get(name)
    if v is None or v == "":
        return None
    try:
        n = int(v)
    except ValueError:
        raise ValueError(f"{name} must be an integer, got {v!r}") from None
    if n not in allowed:
        raise ValueError(f"{name} must be one of {allowed}, got {n}")
    return n


def use_lut() -> bool:
    return _flag("ESCHA_MLX_LUT", False)


def use_exact() -> bool:
    return _flag("ESCHA_HIP_EXACT", False)


def dense_mat() -> bool:
    return _flag("ESCHA_MLX_DENSE_MAT", True)


def block_r_pin() -> int | None:
    return _int("ESCHA_MLX_BLOCK_R", (1, 2, 3, 4, 8, 12, 16))


def dense_block_r_pin() -> int | None:
    return _int("ESCHA_MLX_DENSE_BLOCK_R", (1, 2, 4, 8, 16))
