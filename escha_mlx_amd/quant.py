"""Dense int8 linears (escha_mlx/quant.py): the w8a16 contract of the
checkpoint's ``weight_int8`` [N, K] + per-row ``weight_scale`` [N],

    wf = f16(f32(w8) * f32(scale));  y = f16(f32-accumulated x @ wf^T)

(escha_mlx/quant.py:1-30; CPU statement ref.w8a16, escha_mlx/ref.py:308-311).

The reference repacks the int8 rows into MLX's affine Q8 layout; here the
checkpoint layout is the device layout: ``esc_w8a16`` reads the int8 rows and
the per-row scale directly (16-byte loads, one weight rounded per the contract
before its product).  ``group_size`` is accepted for the call surface and has
no effect: the scale is per output channel, so grouping never changes a value
(escha_mlx/quant.py:27-34).  ``EschaQ8Head`` is the same linear used as the
vocabulary projection (escha_mlx/quant.py:236-251), ``EschaQ8Embedding`` the
token embedding over the same int8 rows (escha_mlx/quant.py:253-266).
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops

DEFAULT_GROUP = 128


class EschaQ8Linear(torch.nn.Module):
    """y = f16(x @ dequant(w)^T), f32 accumulate: the w8a16 contract."""

    def __init__(self, w8, scale, device="cuda") -> None:
        super().__init__()
        w8 = torch.as_tensor(np.asarray(w8, dtype=np.int8)) if not torch.is_tensor(w8) else w8
        scale = (torch.as_tensor(np.asarray(scale, dtype=np.float32)) if not torch.is_tensor(scale)
                 else scale.to(torch.float32))
        if w8.ndim != 2 or w8.dtype != torch.int8 or scale.shape != (w8.shape[0],):
            raise ValueError(f"need int8 [N, K] and scale [N], got {tuple(w8.shape)} / {tuple(scale.shape)}")
        self.w8 = w8.contiguous().to(device)
        self.scale = scale.contiguous().to(device)
        self.out_features, self.in_features = self.w8.shape

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        xf = x.reshape(-1, self.in_features).to(torch.float16).contiguous()
        y = ops.w8a16(xf, self.w8, self.scale)
        return y.reshape(*lead, self.out_features).to(x.dtype)


class EschaQ8Head(EschaQ8Linear):
    """The vocabulary projection (escha_mlx/quant.py:236-251): same contract;
    one to eight flattened rows share each weight row read."""


class EschaQ8Embedding(torch.nn.Module):
    """int8 token embedding (escha_mlx/quant.py:253-266): ids -> f16 rows
    f16(f32(w8[id]) * f32(scale[id])), the contract's dequantised weights."""

    def __init__(self, w8, scale, device="cuda") -> None:
        super().__init__()
        w8 = torch.as_tensor(np.asarray(w8, dtype=np.int8)) if not torch.is_tensor(w8) else w8
        scale = (torch.as_tensor(np.asarray(scale, dtype=np.float32)) if not torch.is_tensor(scale)
                 else scale.to(torch.float32))
        if w8.ndim != 2 or w8.dtype != torch.int8 or scale.shape != (w8.shape[0],):
            raise ValueError(f"need int8 [N, K] and scale [N], got {tuple(w8.shape)} / {tuple(scale.shape)}")
        if w8.shape[1] % 16:
            raise ValueError(f"embedding width {w8.shape[1]} must be a multiple of 16")
        self.w8 = w8.contiguous().to(device)
        self.scale = scale.contiguous().to(device)
        self.num_embeddings, self.embedding_dim = self.w8.shape

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return ops.q8_embed(ids.to(self.w8.device), self.w8, self.scale)


def make_linear(w8: np.ndarray, scale: np.ndarray, group_size: int = DEFAULT_GROUP,
                device="cuda") -> EschaQ8Linear:
    """escha_mlx.quant.make_linear (quant.py:269-279): int8 [N, K] + scale [N]."""
    del group_size  # per-row scale: the group size cannot change a value
    return EschaQ8Linear(w8, scale, device)


def make_head(w8: np.ndarray, scale: np.ndarray, group_size: int = DEFAULT_GROUP,
              device="cuda") -> EschaQ8Head:
    """escha_mlx.quant.make_head (quant.py:282-296)."""
    del group_size
    return EschaQ8Head(w8, scale, device)


def make_embedding(w8: np.ndarray, scale: np.ndarray, group_size: int = DEFAULT_GROUP,
                   device="cuda") -> EschaQ8Embedding:
    """escha_mlx.quant.make_embedding (quant.py:298-308)."""
    del group_size
    return EschaQ8Embedding(w8, scale, device)
