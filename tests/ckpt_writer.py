"""Tiny, format-faithful escha exports for the loader tests, shaped like the
reference's synthetic checkpoints (tests/test_models.py:24-146, 184-288 of the
reference): raw HF tensor names under ``model.language_model.``, E-stacked
expert trios, int8 pairs with f16 scales, f16 router gates, the dense export's
per-linear leaves, and tensors the loader must drop (MTP, vision).

No model skeleton is built on this side, so the f16 remainder is a handful of
representative tensors rather than a whole decoder, and the dense export may
carry projections whose shapes do not match the hidden size (the real 128x128
corners of a shipped linear, whose shipped output pins the loaded module).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

E, H, INTER, VOCAB, LAYERS = 4, 256, 128, 512, 2
PFX = "model.language_model."

MOE_CONFIG = {
    "model_type": "qwen3_5_moe", "hidden_size": H, "num_hidden_layers": LAYERS,
    "num_attention_heads": 4, "num_key_value_heads": 2, "vocab_size": VOCAB,
    "num_experts": E, "num_experts_per_tok": 2, "moe_intermediate_size": INTER,
    "shared_expert_intermediate_size": INTER, "tie_word_embeddings": False,
    "quantization_config": {"quant_method": "eschamoe", "bits": 2.0},
}

DENSE_CONFIG = {
    "model_type": "qwen3_5", "hidden_size": H, "intermediate_size": INTER,
    "num_hidden_layers": LAYERS, "num_attention_heads": 4, "num_key_value_heads": 2,
    "head_dim": 64, "vocab_size": VOCAB, "tie_word_embeddings": False,
    "quantization_config": {"quant_method": "escha", "bits": 2.0},
}


def q8_pair(rng, out_dim, in_dim):
    return (rng.integers(-128, 128, size=(out_dim, in_dim), dtype=np.int8),
            (rng.random(out_dim) * 0.01 + 1e-3).astype(np.float16))


def _code(rng, *shape):
    return rng.integers(-32768, 32768, size=shape, dtype=np.int16)


def _remainder(rng, t):
    """Representative f16 tensors the engine does not own (norms, GDN conv in
    the HF [C, 1, K] layout, attention projections of a non-coded layer)."""
    for i in range(LAYERS):
        t[PFX + f"layers.{i}.input_layernorm.weight"] = (rng.standard_normal(H) * 0.1).astype(np.float16)
        t[PFX + f"layers.{i}.post_attention_layernorm.weight"] = (
            rng.standard_normal(H) * 0.1).astype(np.float16)
    t[PFX + "layers.0.linear_attn.conv1d.weight"] = rng.standard_normal((384, 1, 4)).astype(np.float16)
    t[PFX + "norm.weight"] = (rng.standard_normal(H) * 0.1).astype(np.float16)


def _save(path: Path, t: dict, config: dict, shards: list | None = None) -> None:
    """shards: list of predicates over the tensor name; shard i holds the
    names the i-th predicate accepts first (files read in name order)."""
    from safetensors.numpy import save_file
    path.mkdir(parents=True, exist_ok=True)
    if shards is None:
        save_file(t, str(path / "model.safetensors"))
    else:
        left = dict(t)
        for i, pred in enumerate(shards + [lambda n: True]):
            part = {k: v for k, v in left.items() if pred(k)}
            for k in part:
                del left[k]
            if part:
                save_file(part, str(path / f"model-{i:05d}.safetensors"))
    (path / "config.json").write_text(json.dumps(config))
    qm = config["quantization_config"]
    (path / "quantize_config.json").write_text(json.dumps(qm))


def write_moe_checkpoint(path: Path, rng, shards: int = 1) -> dict:
    """gate_up K=2 and down K=3 expert trios per layer (+ the redundant
    s_in / config leaves), int8 shared expert, f16 gates, int8 embedding /
    head / one attention projection, dropped MTP and vision tensors."""
    t: dict[str, np.ndarray] = {}
    for i in range(LAYERS):
        p = PFX + f"layers.{i}.mlp."
        t[p + "experts.gate_up_proj.escha_code"] = _code(rng, E, H // 16, 2 * INTER // 16, 32)
        # input scales near 1 (as exported) keep the routed outputs in f16's normal range
        t[p + "experts.gate_up_proj.escha_rin"] = rng.standard_normal((E, H)).astype(np.float16)
        t[p + "experts.gate_up_proj.escha_rout"] = (
            rng.standard_normal((E, 2 * INTER)) * 0.05).astype(np.float16)
        t[p + "experts.down_proj.escha_code"] = _code(rng, E, INTER // 16, H // 16, 48)
        t[p + "experts.down_proj.escha_rin"] = rng.standard_normal((E, INTER)).astype(np.float16)
        t[p + "experts.down_proj.escha_rout"] = (rng.standard_normal((E, H)) * 0.05).astype(np.float16)
        t[p + "experts.gate_up_proj.escha_s_in"] = np.ones((E, H), dtype=np.float16)
        t[p + "experts.gate_up_proj.escha_config"] = np.zeros((4,), dtype=np.int32)
        for name, (o, k) in (("gate", (INTER, H)), ("up", (INTER, H)), ("down", (H, INTER))):
            w8, sc = q8_pair(rng, o, k)
            t[p + f"shared_expert.{name}_proj.weight_int8"] = w8
            t[p + f"shared_expert.{name}_proj.weight_scale"] = sc
        t[p + "gate.weight"] = (rng.standard_normal((E, H)) * 0.1).astype(np.float16)
        t[p + "shared_expert_gate.weight"] = (rng.standard_normal((1, H)) * 0.1).astype(np.float16)
    w8, sc = q8_pair(rng, VOCAB, H)
    t[PFX + "embed_tokens.weight_int8"], t[PFX + "embed_tokens.weight_scale"] = w8, sc
    w8, sc = q8_pair(rng, VOCAB, H)
    t["lm_head.weight_int8"], t["lm_head.weight_scale"] = w8, sc
    w8, sc = q8_pair(rng, 512, H)
    t[PFX + "layers.1.self_attn.q_proj.weight_int8"] = w8
    t[PFX + "layers.1.self_attn.q_proj.weight_scale"] = sc
    t["mtp.head.weight"] = np.zeros((4, 4), dtype=np.float16)
    t["model.visual.patch_embed.weight"] = np.zeros((4, 4), dtype=np.float16)
    _remainder(rng, t)
    split = None
    if shards > 1:
        split = [lambda n, i=i: f"layers.{i}." in n for i in range(shards - 1)]
    _save(path, t, MOE_CONFIG, split)
    return t


#: coded projections of the dense export and their rates (K=3 for the wide
#: MLP legs, K=2 elsewhere, as shipped): name -> (IC, OC, K)
DENSE_PROJ = {
    "layers.0.linear_attn.in_proj_qkv": (H, 384, 2),
    "layers.0.linear_attn.in_proj_z": (H, 128, 2),
    "layers.0.linear_attn.out_proj": (128, H, 2),
    "layers.1.self_attn.q_proj": (H, H, 2),
    "layers.1.self_attn.k_proj": (H, 128, 2),
    "layers.1.self_attn.v_proj": (H, 128, 2),
    "layers.1.self_attn.o_proj": (H, H, 2),
    "layers.0.mlp.gate_proj": (H, INTER, 2),
    "layers.0.mlp.up_proj": (H, INTER, 3),
    "layers.0.mlp.down_proj": (INTER, H, 3),
}
#: projections that carry the real corners of a shipped linear instead
REAL_CORNERS = {"layers.1.mlp.gate_proj": "k2", "layers.1.mlp.up_proj": "k3"}


def write_dense_checkpoint(path: Path, rng, corners: dict | None = None, optional: bool = True,
                           leaf_shards: bool = True) -> dict:
    """Every projection coded (leaves per linear), real corners at
    REAL_CORNERS when ``corners`` (tag -> golden dict) is given, int8
    embedding / head.  ``optional=False`` leaves out s_in / s_out / config /
    bias.  ``leaf_shards`` writes one shard per leaf kind, codes last, so the
    stream arrives grouped by leaf as a real dense export does."""
    t: dict[str, np.ndarray] = {}
    for base, (ic, oc, K) in DENSE_PROJ.items():
        p = PFX + base
        t[p + ".escha_code"] = _code(rng, ic // 16, oc // 16, 16 * K)
        t[p + ".escha_rin"] = (rng.standard_normal(ic) * 0.05).astype(np.float16)
        t[p + ".escha_rout"] = (rng.standard_normal(oc) * 0.05).astype(np.float16)
        if optional:
            t[p + ".escha_s_in"] = (1.0 + rng.standard_normal(ic) * 0.01).astype(np.float32)
            t[p + ".escha_s_out"] = (1.0 + rng.standard_normal(oc) * 0.01).astype(np.float32)
            t[p + ".escha_config"] = np.array([16, K, 2, 1, ic, oc], dtype=np.int32)
            t[p + ".bias"] = (rng.standard_normal(oc) * 0.005).astype(np.float16)
    for base, tag in (REAL_CORNERS.items() if corners else ()):
        g, p = corners[tag], PFX + base
        t[p + ".escha_code"], t[p + ".escha_rin"], t[p + ".escha_rout"] = g["code"], g["rin"], g["rout"]
        t[p + ".escha_s_in"], t[p + ".escha_s_out"], t[p + ".bias"] = g["s_in"], g["s_out"], g["bias"]
        t[p + ".escha_config"] = np.array([16, g["K"], 2, 1, 128, 128], dtype=np.int32)
    w8, sc = q8_pair(rng, VOCAB, H)
    t[PFX + "embed_tokens.weight_int8"], t[PFX + "embed_tokens.weight_scale"] = w8, sc
    w8, sc = q8_pair(rng, VOCAB, H)
    t["lm_head.weight_int8"], t["lm_head.weight_scale"] = w8, sc
    t[PFX + "layers.0.linear_attn.in_proj_a.weight"] = (rng.standard_normal((4, H)) * 0.1).astype(np.float16)
    t["mtp.head.weight"] = np.zeros((4, 4), dtype=np.float16)
    t["model.visual.patch_embed.weight"] = np.zeros((4, 4), dtype=np.float16)
    _remainder(rng, t)
    split = None
    if leaf_shards:
        split = [lambda n, lf=lf: n.endswith(lf) for lf in
                 (".escha_s_in", ".escha_s_out", ".escha_config", ".bias", ".escha_rin",
                  ".escha_rout")] + [lambda n: not n.endswith(".escha_code")]
    _save(path, t, DENSE_CONFIG, split)
    return t


def reload(path: Path) -> dict:
    """Every tensor of a written checkpoint, for read-modify-rewrite tests."""
    from safetensors import safe_open
    out = {}
    for f in sorted(path.glob("*.safetensors")):
        with safe_open(str(f), framework="numpy") as h:
            out.update({k: h.get_tensor(k) for k in h.keys()})
    return out


def rewrite(path: Path, t: dict) -> None:
    """Replace the checkpoint's shards with one holding ``t``."""
    from safetensors.numpy import save_file
    for f in path.glob("*.safetensors"):
        f.unlink()
    save_file(t, str(path / "model.safetensors"))
