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
  quant  — escha_mlx.quant's int8 modules (EschaQ8Linear / Head / Embedding)
  loader — escha_mlx.loader + the architecture plugins' checkpoint loaders
           (load_model, resolve, is_escha_checkpoint, LastPositionHead)
"""
from . import _lib, dense, envs, loader, moe, ops, quant  # noqa: F401

__all__ = ["ops", "dense", "moe", "quant", "loader", "envs"]
__version__ = "0.1.0"
