"""Load an escha checkpoint onto the GPU: the on-disk format and the repack at
load (escha_mlx/loader.py:1-223 and the two architecture plugins'
CheckpointLoader, escha_mlx/models/qwen3_5_moe.py:276-406,
escha_mlx/models/qwen3_5.py:200-361).

The export is a directory of safetensors shards plus config.json, read one
tensor at a time (loader.py:47-57) and converted to its device form as soon as
its group allows, so host memory never holds the coded body twice:

  * eschamoe (model_type qwen3_5_moe): routed experts as E-stacked trios
    ``layers.N.mlp.experts.{gate_up_proj,down_proj}.escha_{code,rin,rout}``
    (``escha_s_in`` / ``escha_s_out`` / ``escha_config`` are redundant there and
    dropped); int8 ``weight_int8`` + ``weight_scale`` pairs for the shared
    expert, other dense linears, the embedding and the head; the f16 router
    ``mlp.gate.weight`` and ``mlp.shared_expert_gate.weight``.  Each layer's
    experts, shared expert and gates become one ``moe.EschaSparseMoeBlock``.
  * escha (model_type qwen3_5): every projection coded, the leaves of one
    linear ``escha_code`` / ``escha_rin`` / ``escha_rout`` (+ optional
    ``escha_s_in`` / ``escha_s_out`` / ``escha_config`` / ``bias``) spread over
    the whole stream, since the export groups tensors by leaf name.  Codes are
    packed to device words on arrival; each linear is assembled in finalize
    (``dense.build``: scales folded at load, config cross-checked).

What the reference hands to mlx-lm (its model skeleton, attention and GDN
layers, and the sanitize of the f16 remainder) is outside this engine: the
f16 remainder comes back unchanged under its original names in
``LoadedCheckpoint.tensors`` for the caller's own skeleton, and the built
modules in ``LoadedCheckpoint.modules`` under the skeleton paths the reference
installs them at (``layers.N.mlp``, ``layers.N.self_attn.q_proj``,
``embed_tokens``, ``lm_head``).  Apple's wired-memory policy
(loader.py:59-101) has no counterpart: device memory is allocated, not wired.
"""
from __future__ import annotations

import glob
import json
import os
from pathlib import Path

import numpy as np
import torch

from . import dense, envs, moe, quant

#: quant_method values this runtime loads (loader.py:29-34).
QUANT_METHODS = frozenset({"escha", "eschamoe"})
LM_PREFIX = "model.language_model."


def is_escha_checkpoint(path) -> bool:
    """quant_method from quantize_config.json or config.json's
    quantization_config (loader.py:37-45)."""
    path = Path(path)
    for fname in ("quantize_config.json", "config.json"):
        f = path / fname
        if f.exists():
            cfg = json.loads(f.read_text())
            qc = cfg if fname == "quantize_config.json" else cfg.get("quantization_config", {})
            if qc.get("quant_method") in QUANT_METHODS:
                return True
    return False


def iter_tensors(path):
    """(name, numpy array) one tensor at a time over the sorted shards (loader.py:47-57)."""
    from safetensors import safe_open
    shards = sorted(glob.glob(str(Path(path) / "*.safetensors")))
    if not shards:
        raise FileNotFoundError(f"no safetensors shards under {path}")
    for shard in shards:
        with safe_open(shard, framework="numpy") as f:
            for name in f.keys():
                yield name, f.get_tensor(name)


def strip_lm_prefix(name: str) -> str:
    """Drop the VLM wrapper prefix of language-model tensors (loader.py:60-62)."""
    return name[len(LM_PREFIX):] if name.startswith(LM_PREFIX) else name


def _dropped(name: str) -> bool:
    """MTP and vision tensors are not part of the decoder (qwen3_5_moe.py:324-326)."""
    return name.startswith("mtp.") or ".visual." in name or name.startswith("visual.")


def use_last_logit() -> bool:
    """ESCHA_MLX_LAST_LOGIT (default 1): the head sees the final position only
    (loader.py:135-138)."""
    return envs.parse_bool("ESCHA_MLX_LAST_LOGIT", True)


def q8_group() -> int:
    """ESCHA_MLX_Q8_GROUP (default 128): accepted for the call surface; a
    per-row scale makes the group size irrelevant to every value."""
    v = os.environ.get("ESCHA_MLX_Q8_GROUP", "")
    if v == "":
        return quant.DEFAULT_GROUP
    try:
        n = int(v)
    except ValueError:
        raise ValueError(f"ESCHA_MLX_Q8_GROUP must be a positive integer, got {v!r}") from None
    if n <= 0:
        raise ValueError(f"ESCHA_MLX_Q8_GROUP must be a positive integer, got {v!r}")
    return n


class LastPositionHead(torch.nn.Module):
    """Apply the head to the last position of a [B, S, H] input only
    (loader.py:104-132): [B, S, H] -> [B, 1, V]."""

    def __init__(self, inner: torch.nn.Module) -> None:
        super().__init__()
        self.inner = inner

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.ndim == 3 and x.shape[1] > 1:
            x = x[:, -1:, :]
        return self.inner(x)


class LoadedCheckpoint:
    """What a load produces: the built modules by skeleton path, the f16
    remainder by original tensor name, and the load's counts."""

    def __init__(self, config: dict, model_type: str) -> None:
        self.config, self.model_type = config, model_type
        self.modules: dict[str, torch.nn.Module] = {}
        self.tensors: dict[str, np.ndarray] = {}
        self.escha_arrays: list[torch.Tensor] = []
        self.n_layers = self.n_coded = self.n_q8 = self.n_bias = self.dropped = self.n_fused = 0
        self.rates: dict[int, int] = {}

    def __getitem__(self, path: str) -> torch.nn.Module:
        return self.modules[path]

    def coded_bytes(self) -> int:
        """Bytes of the coded streams and their transform vectors on the device."""
        return sum(t.numel() * t.element_size() for t in self.escha_arrays)


def _text_config(config: dict) -> dict:
    return config.get("text_config", config)


def _check_layer(base: str, n_layers: int) -> None:
    """A module path under ``layers.N`` must name a layer of the decoder."""
    idx = base.split(".")[1]
    if not idx.isdigit() or int(idx) >= n_layers:
        raise ValueError(f"{base}: outside the decoder stack of {n_layers} layers")


class _Q8Mixin:
    """int8 pair streaming shared by both plugins (qwen3_5_moe.py:304-321)."""

    def _q8_pair(self, base: str, leaf: str, w: np.ndarray) -> None:
        pair = self._int8_np.setdefault(base, {})
        pair[leaf] = w
        if len(pair) == 2:
            self._install_q8(base, pair)
            del self._int8_np[base]

    def _install_q8(self, base: str, pair: dict) -> None:
        w8, scale = pair["weight_int8"], pair["weight_scale"]
        ck, g, dev = self.ckpt, self.group_size, self.device
        if base == "lm_head":
            head = quant.make_head(w8, scale, g, dev)
            ck.modules["lm_head"] = LastPositionHead(head) if use_last_logit() else head
        elif base == "embed_tokens":
            ck.modules["embed_tokens"] = quant.make_embedding(w8, scale, g, dev)
        elif base.startswith("layers."):
            _check_layer(base, self.n_layers)
            ck.modules[base] = quant.make_linear(w8, scale, g, dev)
        else:
            raise ValueError(f"unexpected int8 tensor: {base}")
        ck.n_q8 += 1

    def _check_pairs(self) -> None:
        if self._int8_np:
            raise ValueError("incomplete int8 tensor pairs: "
                             f"{ {k: sorted(v) for k, v in self._int8_np.items()} }")


class MoECheckpointLoader(_Q8Mixin):
    """eschamoe / qwen3_5_moe exports (qwen3_5_moe.py:276-406)."""

    MODEL_TYPE = "qwen3_5_moe"
    _DROP_LEAVES = frozenset({"escha_s_in", "escha_s_out", "escha_config"})
    _EXPERT_LEAVES = ("escha_code", "escha_rin", "escha_rout")

    def __init__(self, config: dict, group_size: int, device="cuda") -> None:
        tc = _text_config(config)
        self.group_size, self.device = group_size, device
        self.ckpt = LoadedCheckpoint(config, self.MODEL_TYPE)
        self.n_layers = int(tc["num_hidden_layers"])
        self.top_k = int(tc["num_experts_per_tok"])
        self.hidden_size = int(tc["hidden_size"])
        self.num_experts = int(tc["num_experts"])
        self._experts_np: dict[tuple[int, str], dict[str, np.ndarray]] = {}
        self._experts: dict[tuple[int, str], moe.EschaExperts] = {}
        self._int8_np: dict[str, dict[str, np.ndarray]] = {}
        self._shared_np: dict[str, dict[str, np.ndarray]] = {}
        self._gates: dict[tuple[int, str], np.ndarray] = {}

    def consume(self, name: str, w: np.ndarray) -> None:
        if _dropped(name):
            self.ckpt.dropped += 1
            return
        s = strip_lm_prefix(name)
        parts = s.split(".")
        if ".mlp.experts." in s:
            layer, proj, leaf = int(parts[1]), parts[4], parts[5]
            if leaf in self._DROP_LEAVES:
                self.ckpt.dropped += 1
                return
            if leaf not in self._EXPERT_LEAVES:
                raise ValueError(f"{name}: unknown expert tensor {leaf!r}")
            group = self._experts_np.setdefault((layer, proj), {})
            group[leaf] = w
            if len(group) == len(self._EXPERT_LEAVES):
                # the trio is complete: upload it and drop the host copy
                self._experts[(layer, proj)] = moe.EschaExperts(
                    group["escha_code"], group["escha_rin"], group["escha_rout"], self.device)
                del self._experts_np[(layer, proj)]
            return
        if s.endswith(".weight_int8") or s.endswith(".weight_scale"):
            base, leaf = s.rsplit(".", 1)
            if ".shared_expert." in s:
                self._shared_np.setdefault(base, {})[leaf] = w
            else:
                self._q8_pair(base, leaf, w)
            return
        if s.endswith(".mlp.gate.weight") or s.endswith(".mlp.shared_expert_gate.weight"):
            self._gates[(int(parts[1]), parts[3])] = w
            return
        self.ckpt.tensors[name] = w

    def finalize(self) -> LoadedCheckpoint:
        if self._experts_np:
            raise ValueError("incomplete expert tensors: "
                             f"{ {k: sorted(v) for k, v in self._experts_np.items()} }")
        self._check_pairs()
        ck = self.ckpt
        for i in range(self.n_layers):
            try:
                gu = self._experts.pop((i, "gate_up_proj"))
                dn = self._experts.pop((i, "down_proj"))
                pref = f"layers.{i}.mlp.shared_expert"
                shared = {}
                for p in ("gate", "up", "down"):
                    pair = self._shared_np.pop(f"{pref}.{p}_proj")
                    shared[f"{p}_w8"], shared[f"{p}_scale"] = pair["weight_int8"], pair["weight_scale"]
                gate_w = self._gates.pop((i, "gate"))
                shg_w = self._gates.pop((i, "shared_expert_gate"))
            except KeyError as e:
                raise ValueError(f"layer {i}: MoE block tensor missing ({e.args[0]})") from None
            ck.modules[f"layers.{i}.mlp"] = moe.EschaSparseMoeBlock(
                self.hidden_size, self.num_experts, self.top_k, gu, dn, gate_w, shg_w, shared,
                self.group_size, self.device)
            ck.escha_arrays += gu.arrays() + dn.arrays()
            for k in (gu.K, dn.K):
                ck.rates[k] = ck.rates.get(k, 0) + 1
        left = list(self._experts) + list(self._shared_np) + list(self._gates)
        if left:
            raise ValueError(f"tensors beyond num_hidden_layers={self.n_layers}: {left[:4]}")
        ck.n_layers = self.n_layers
        return ck


class DenseCheckpointLoader(_Q8Mixin):
    """escha / qwen3_5 exports, every projection coded (qwen3_5.py:200-361)."""

    MODEL_TYPE = "qwen3_5"

    def __init__(self, config: dict, group_size: int, device="cuda") -> None:
        self.group_size, self.device = group_size, device
        self.ckpt = LoadedCheckpoint(config, self.MODEL_TYPE)
        self.n_layers = int(_text_config(config)["num_hidden_layers"])
        self._coded: dict[str, dict[str, object]] = {}
        self._bias: dict[str, tuple[str, np.ndarray]] = {}
        self._int8_np: dict[str, dict[str, np.ndarray]] = {}

    def consume(self, name: str, w: np.ndarray) -> None:
        if _dropped(name):
            self.ckpt.dropped += 1
            return
        s = strip_lm_prefix(name)
        base, _, leaf = s.rpartition(".")
        if leaf in dense.LEAVES and leaf != "bias":
            group = self._coded.setdefault(base, {})
            # the code streams are the bulk of the export: packed to the
            # device on arrival, so no host copy outlives its tensor
            group[leaf] = dense.pack_code(w, self.device) if leaf == "escha_code" else w
            return
        if leaf.startswith("escha_"):
            raise ValueError(
                f"{name}: unknown escha tensor {leaf!r}. This export uses a format feature "
                f"this runtime does not implement (known leaves: {sorted(dense.LEAVES)}).")
        if leaf == "bias":
            self._bias[base] = (name, w)
            return
        if leaf in ("weight_int8", "weight_scale"):
            self._q8_pair(base, leaf, w)
            return
        self.ckpt.tensors[name] = w

    def finalize(self) -> LoadedCheckpoint:
        self._check_pairs()
        ck = self.ckpt
        for base in sorted(self._coded):
            group = self._coded[base]
            missing = dense.REQUIRED - set(group)
            if missing:
                raise ValueError(f"{base}: incomplete escha linear, missing {sorted(missing)}")
            if not base.startswith("layers."):
                raise ValueError(f"coded linear outside the decoder stack: {base}")
            _check_layer(base, self.n_layers)
            held = self._bias.pop(base, None)
            if held is not None:
                group["bias"] = held[1]
                ck.n_bias += 1
            lin = dense.build(group, self.device)
            ck.modules[base] = lin
            ck.rates[lin.K] = ck.rates.get(lin.K, 0) + 1
            ck.escha_arrays += lin._w.arrays()
            ck.n_coded += 1
        self._coded.clear()
        # a bias no coded linear claimed belongs to an ordinary module
        for orig, w in self._bias.values():
            ck.tensors[orig] = w
        self._bias.clear()
        ck.n_layers = self.n_layers
        install_projection_fusion(ck)
        return ck


def install_projection_fusion(ck: LoadedCheckpoint) -> int:
    """One dispatch per projection pair of each decoder layer
    (escha_mlx/models/qwen3_5.py:173-198): ``layers.N.mlp`` becomes a
    ``dense.EschaMLP`` over coded gate/up/down, ``layers.N.self_attn.kv`` a
    ``dense.EschaKVProjection`` over coded k/v.  The projections stay
    available under their own paths.  Returns the number of groups installed."""
    installed = 0
    for i in range(ck.n_layers):
        p = f"layers.{i}."
        mlp = [ck.modules.get(p + f"mlp.{n}_proj") for n in ("gate", "up", "down")]
        if all(isinstance(m, dense.EschaLinear) for m in mlp) and not isinstance(
                ck.modules.get(p + "mlp"), dense.EschaMLP):
            ck.modules[p + "mlp"] = dense.EschaMLP(*mlp)
            installed += 1
        kv = [ck.modules.get(p + f"self_attn.{n}_proj") for n in ("k", "v")]
        if all(isinstance(m, dense.EschaLinear) for m in kv) and p + "self_attn.kv" not in ck.modules:
            ck.modules[p + "self_attn.kv"] = dense.EschaKVProjection(*kv)
            installed += 1
    ck.n_fused = installed
    return installed


#: model_type -> plugin (escha_mlx/models/__init__.py:36-50).
REGISTRY = {
    MoECheckpointLoader.MODEL_TYPE: MoECheckpointLoader,
    DenseCheckpointLoader.MODEL_TYPE: DenseCheckpointLoader,
}


def resolve(config: dict):
    """The plugin for this checkpoint's model_type (models/__init__.py:43-50)."""
    model_type = config.get("model_type")
    if model_type not in REGISTRY:
        raise ValueError(f"escha_mlx_amd: unsupported model_type {model_type!r} — supported: "
                         f"{sorted(REGISTRY)}")
    return REGISTRY[model_type]


def load_model(path, *, device="cuda") -> LoadedCheckpoint:
    """Stream a checkpoint through its plugin (loader.py:141-186)."""
    path = Path(path)
    if not is_escha_checkpoint(path):
        raise ValueError(f"{path} is not an escha checkpoint (expected quantization_config."
                         f"quant_method in {sorted(QUANT_METHODS)})")
    config = json.loads((path / "config.json").read_text())
    plugin = resolve(config)(config, q8_group(), device)
    for name, w in iter_tensors(path):
        plugin.consume(name, w)
    return plugin.finalize()
