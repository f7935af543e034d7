"""Loader on the CPU: format detection, registry, streaming grouping, the
repack at load and every rejection the reference's loader makes
(tests/test_models.py:50-58, 148-433 of the reference), on tiny synthetic
exports written with safetensors.  Modules are built on device "cpu" (their
construction is host work; forward passes are GPU tests)."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from . import ckpt_writer as W


def _loader():
    from escha_mlx_amd import loader
    return loader


@pytest.mark.parametrize("model_type", ["qwen3_5_moe", "qwen3_5"])
def test_resolve_known_and_unknown(model_type):
    L = _loader()
    assert L.resolve({"model_type": model_type}).MODEL_TYPE == model_type
    with pytest.raises(ValueError, match="qwen3_5_moe"):
        L.resolve({"model_type": "made_up_arch"})


def test_is_escha_checkpoint(tmp_path):
    L = _loader()
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": {"quant_method": "escha"}}))
    assert L.is_escha_checkpoint(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": {"quant_method": "gptq"}}))
    assert not L.is_escha_checkpoint(tmp_path)
    (tmp_path / "quantize_config.json").write_text(json.dumps({"quant_method": "eschamoe"}))
    assert L.is_escha_checkpoint(tmp_path)
    with pytest.raises(ValueError, match="not an escha checkpoint"):
        L.load_model(tmp_path / "missing", device="cpu")


@pytest.mark.parametrize("shards", [1, 2])
def test_moe_checkpoint_structure_and_repack(tmp_path, shards):
    from escha_mlx_amd import moe, ops, quant
    L = _loader()
    t = W.write_moe_checkpoint(tmp_path, np.random.default_rng(0), shards=shards)
    ck = L.load_model(tmp_path, device="cpu")
    assert ck.model_type == "qwen3_5_moe" and ck.n_layers == W.LAYERS
    for i in range(W.LAYERS):
        blk = ck[f"layers.{i}.mlp"]
        assert isinstance(blk, moe.EschaSparseMoeBlock)
        p = W.PFX + f"layers.{i}.mlp."
        gu, dn = blk.experts._gu, blk.experts._dn
        assert (gu.K, dn.K) == (2, 3)
        # repack: int16 export -> little-endian u32 words, rin/rout f16 -> f32
        want = ops.code_to_u32(t[p + "experts.gate_up_proj.escha_code"]).view(np.int32)
        assert np.array_equal(gu.code.numpy(), want)
        assert np.array_equal(dn.rout.numpy(), t[p + "experts.down_proj.escha_rout"].astype(np.float32))
        assert np.array_equal(blk.gate_w.numpy(), t[p + "gate.weight"])
        assert np.array_equal(blk.shg_w.numpy(), t[p + "shared_expert_gate.weight"])
        assert np.array_equal(blk.sh_down.w8.numpy(), t[p + "shared_expert.down_proj.weight_int8"])
        assert np.array_equal(blk.sh_up.scale.numpy(),
                              t[p + "shared_expert.up_proj.weight_scale"].astype(np.float32))
    assert isinstance(ck["embed_tokens"], quant.EschaQ8Embedding)
    assert isinstance(ck["layers.1.self_attn.q_proj"], quant.EschaQ8Linear)
    head = ck["lm_head"]
    assert isinstance(head, L.LastPositionHead) and isinstance(head.inner, quant.EschaQ8Head)
    # counts: q_proj + embed + head; dropped = mtp + visual + 2 redundant leaves per layer
    assert ck.n_q8 == 3 and ck.dropped == 2 + 2 * W.LAYERS
    assert ck.rates == {2: W.LAYERS, 3: W.LAYERS}
    # the f16 remainder comes back untouched under its original names
    rem = {k for k in t if k.endswith("layernorm.weight") or k.endswith("norm.weight")
           or k.endswith("conv1d.weight")}
    assert set(ck.tensors) == rem
    for k in rem:
        assert ck.tensors[k].dtype == t[k].dtype and np.array_equal(ck.tensors[k], t[k])
    assert ck.coded_bytes() == sum(a.numel() * a.element_size() for a in ck.escha_arrays) > 0


def test_moe_experts_upload_when_trio_completes(tmp_path):
    """The streaming contract: an expert trio leaves host memory the moment its
    third leaf arrives (qwen3_5_moe.py:292-300, 334-344)."""
    L = _loader()
    t = W.write_moe_checkpoint(tmp_path, np.random.default_rng(1))
    cfg = json.loads((tmp_path / "config.json").read_text())
    plug = L.resolve(cfg)(cfg, 128, "cpu")
    p = W.PFX + "layers.0.mlp.experts.down_proj."
    plug.consume(p + "escha_code", t[p + "escha_code"])
    plug.consume(p + "escha_rin", t[p + "escha_rin"])
    assert (0, "down_proj") in plug._experts_np and not plug._experts
    plug.consume(p + "escha_rout", t[p + "escha_rout"])
    assert not plug._experts_np and (0, "down_proj") in plug._experts


def test_last_logit_off_gives_the_bare_head(tmp_path, monkeypatch):
    from escha_mlx_amd import quant
    L = _loader()
    W.write_moe_checkpoint(tmp_path, np.random.default_rng(2))
    monkeypatch.setenv("ESCHA_MLX_LAST_LOGIT", "0")
    assert isinstance(L.load_model(tmp_path, device="cpu")["lm_head"], quant.EschaQ8Head)
    monkeypatch.setenv("ESCHA_MLX_LAST_LOGIT", "maybe")
    with pytest.raises(ValueError, match="ESCHA_MLX_LAST_LOGIT"):
        L.load_model(tmp_path, device="cpu")


def test_moe_checkpoint_rejections(tmp_path):
    L = _loader()
    W.write_moe_checkpoint(tmp_path, np.random.default_rng(3))
    good = W.reload(tmp_path)
    cases = [
        (lambda t: t.pop(W.PFX + "layers.1.mlp.experts.down_proj.escha_rin"), "incomplete expert tensors"),
        (lambda t: t.pop("lm_head.weight_scale"), "incomplete int8 tensor pairs"),
        (lambda t: t.pop(W.PFX + "layers.0.mlp.shared_expert_gate.weight"), "layer 0: MoE block tensor missing"),
        (lambda t: t.__setitem__(W.PFX + "layers.0.mlp.experts.down_proj.escha_theta",
                                 np.zeros(4, np.int8)), "unknown expert tensor"),
        (lambda t: t.__setitem__("model.foo.weight_int8", np.zeros((4, 16), np.int8))
         or t.__setitem__("model.foo.weight_scale", np.ones(4, np.float16)), "unexpected int8 tensor"),
    ]
    for mutate, msg in cases:
        t = dict(good)
        mutate(t)
        W.rewrite(tmp_path, t)
        with pytest.raises(ValueError, match=msg):
            L.load_model(tmp_path, device="cpu")


@pytest.mark.parametrize("leaf_shards", [True, False])
def test_dense_checkpoint_structure_and_fold(tmp_path, monkeypatch, leaf_shards):
    from escha_mlx_amd import dense, quant
    L = _loader()
    monkeypatch.setenv("ESCHA_MLX_BIAS", "1")
    t = W.write_dense_checkpoint(tmp_path, np.random.default_rng(4), corners=real_corners(),
                                 leaf_shards=leaf_shards)
    ck = L.load_model(tmp_path, device="cpu")
    assert ck.model_type == "qwen3_5" and ck.n_coded == len(W.DENSE_PROJ) + 2
    for base, (ic, oc, K) in W.DENSE_PROJ.items():
        lin = ck[base]
        assert isinstance(lin, dense.EschaLinear) and lin.K == K and lin.bias is not None
        p = W.PFX + base
        # fold at load: rin * s_in and rout * s_out in float32 (ref.py:242-277)
        ri, ro = R.fold_scales(t[p + ".escha_rin"], t[p + ".escha_rout"], t[p + ".escha_s_in"],
                               t[p + ".escha_s_out"])
        assert np.array_equal(lin._w.rin.numpy(), ri) and np.array_equal(lin._w.rout.numpy(), ro)
        assert np.array_equal(lin.bias.numpy(), t[p + ".bias"])
    assert ck.rates == {2: 8 + 1, 3: 2 + 1}
    assert isinstance(ck["embed_tokens"], quant.EschaQ8Embedding)
    assert ck.n_bias == len(W.DENSE_PROJ) + 2
    assert ck.dropped == 2
    assert W.PFX + "layers.0.linear_attn.in_proj_a.weight" in ck.tensors
    # projection fusion (qwen3_5.py:173-198): layer 0's coded MLP, layer 1's k/v
    assert isinstance(ck["layers.0.mlp"], dense.EschaMLP)
    assert ck["layers.0.mlp"].up_proj is ck["layers.0.mlp.up_proj"]
    kv = ck["layers.1.self_attn.kv"]
    assert isinstance(kv, dense.EschaKVProjection) and kv.v_proj is ck["layers.1.self_attn.v_proj"]
    assert "layers.1.mlp" not in ck.modules and ck.n_fused == 2


def real_corners():
    """Both real 128x128 corners of shipped linears (reference
    tests/data/qwen3_5/lin_k{2,3}_*), keyed by tag."""
    from .conftest import GOLDEN

    def rd(tag, sfx, dt, shape):
        return np.fromfile(GOLDEN / "qwen3_5" / f"lin_{tag}_{sfx}", dtype=dt).reshape(shape)
    out = {}
    for tag, K in (("k2", 2), ("k3", 3)):
        out[tag] = {"K": K, "code": rd(tag, "code.i16", np.int16, (8, 8, 16 * K)),
                    "rin": rd(tag, "rin.f16", np.float16, (128,)),
                    "rout": rd(tag, "rout.f16", np.float16, (128,)),
                    "s_in": rd(tag, "s_in.f32", np.float32, (128,)),
                    "s_out": rd(tag, "s_out.f32", np.float32, (128,)),
                    "bias": rd(tag, "bias.f16", np.float16, (128,)),
                    "x": rd(tag, "x.f16", np.float16, (8, 128)),
                    "deploy": rd(tag, "deploy.f16", np.float16, (8, 128))}
    return out


def test_dense_checkpoint_bias_default_off_and_optional_leaves(tmp_path, monkeypatch):
    L = _loader()
    monkeypatch.delenv("ESCHA_MLX_BIAS", raising=False)
    W.write_dense_checkpoint(tmp_path / "a", np.random.default_rng(5))
    ck = L.load_model(tmp_path / "a", device="cpu")
    assert all(ck[b].bias is None for b in W.DENSE_PROJ) and ck.n_bias == len(W.DENSE_PROJ)
    monkeypatch.setenv("ESCHA_MLX_BIAS", "1")
    t = W.write_dense_checkpoint(tmp_path / "b", np.random.default_rng(6), optional=False)
    ck = L.load_model(tmp_path / "b", device="cpu")
    for base in W.DENSE_PROJ:
        lin = ck[base]
        assert lin.bias is None
        p = W.PFX + base
        assert np.array_equal(lin._w.rin.numpy(), t[p + ".escha_rin"].astype(np.float32))


def test_dense_checkpoint_rejections(tmp_path):
    L = _loader()
    W.write_dense_checkpoint(tmp_path, np.random.default_rng(7))
    good = W.reload(tmp_path)
    q = W.PFX + "layers.0.mlp.gate_proj"
    cases = [
        (lambda t: t.pop(q + ".escha_rout"), "incomplete escha linear"),
        (lambda t: t.__setitem__(q + ".escha_rotation_theta", np.zeros((4, 4), np.int8)),
         "unknown escha tensor"),
        (lambda t: t.pop(W.PFX + "embed_tokens.weight_int8"), "incomplete int8 tensor pairs"),
        (lambda t: t.__setitem__(q + ".escha_config", np.array([16, 3, 2, 1, 256, 128], np.int32)),
         "disagrees with the code stream"),
        (lambda t: t.__setitem__(q + ".escha_config", np.array([16, 2, 2, 7, 256, 128], np.int32)),
         "codebook id 7"),
        (lambda t: t.__setitem__(q + ".escha_s_in", np.ones((2, 256), np.float32)), "escha_s_in"),
        (lambda t: t.__setitem__(q + ".escha_code", np.zeros((16, 8, 64), np.int16)), "K=4"),
        (lambda t: [t.__setitem__(W.PFX + "layers.5.mlp.gate_proj" + k[len(q):], v)
                    for k, v in list(t.items()) if k.startswith(q + ".")], "outside the decoder stack"),
        (lambda t: [t.__setitem__("model.foo" + k[len(q):], v)
                    for k, v in list(t.items()) if k.startswith(q + ".")], "outside the decoder stack"),
    ]
    for mutate, msg in cases:
        t = dict(good)
        mutate(t)
        W.rewrite(tmp_path, t)
        with pytest.raises(ValueError, match=msg):
            L.load_model(tmp_path, device="cpu")


def test_unclaimed_bias_returns_to_the_remainder(tmp_path):
    L = _loader()
    W.write_dense_checkpoint(tmp_path, np.random.default_rng(8))
    t = W.reload(tmp_path)
    name = W.PFX + "layers.0.linear_attn.in_proj_a.bias"
    t[name] = np.ones(4, np.float16)
    W.rewrite(tmp_path, t)
    ck = L.load_model(tmp_path, device="cpu")
    assert name in ck.tensors and np.array_equal(ck.tensors[name], t[name])


def test_q8_group_env(monkeypatch):
    L = _loader()
    monkeypatch.setenv("ESCHA_MLX_Q8_GROUP", "64")
    assert L.q8_group() == 64
    monkeypatch.setenv("ESCHA_MLX_Q8_GROUP", "0")
    with pytest.raises(ValueError, match="ESCHA_MLX_Q8_GROUP"):
        L.q8_group()


def test_embedding_rejects_bad_width():
    from escha_mlx_amd import quant
    with pytest.raises(ValueError, match="multiple of 16"):
        quant.make_embedding(np.zeros((4, 24), np.int8), np.ones(4, np.float16), device="cpu")
    emb = quant.make_embedding(np.zeros((4, 32), np.int8), np.ones(4, np.float16), device="cpu")
    with pytest.raises(ValueError, match="GPU tensors"):
        emb(torch.tensor([0, 1]))
