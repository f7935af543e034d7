"""escha_mlx_amd — MI355X-native engine for escha-mlx's coded-projection hot path.

Trellis-codec weight decode (hash and table variants, fixed f16 rounding
points) fused with the random-sign 128-point Hadamard transforms and the
GEMV / row-blocked GEMM over the decoded weights, plus the routed-MoE expert
path — hand-written HIP for gfx950 behind a C ABI (include/escha_hip.h),
reached from Python through ctypes with the reference's call surface:

  ops    — escha_mlx.msl kernel wrappers (decode_tiles, moe_gemv, scaled_had, ...)
  dense  — escha_mlx.dense (EschaWeight, EschaLinear, build, pack_code, ...)
  moe    — escha_mlx.moe (EschaExperts, build_groups, ...) + the expert path
           and the whole MoE block (router, shared expert)
  quant  — escha_mlx.quant's w8a16 linears (EschaQ8Linear, make_linear, ...)
"""
from . import _lib, dense, envs, moe, ops, quant  # noqa: F401

__all__ = ["ops", "dense", "moe", "quant", "envs"]
__version__ = "0.1.0"
