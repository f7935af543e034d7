"""Loaded checkpoints run on the GPU (the reference's end-to-end checkpoint
tests, tests/test_models.py:148-180, 291-335, restated for the modules this
engine owns): each MoE block of a tiny eschamoe export against the oracle's
full block on the same tensors, the int8 embedding bit-exact, the head on the
last position, and a dense export whose two real corners must reproduce the
shipped ``deploy`` outputs after the loader folds their scales."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from . import ckpt_writer as W
from .conftest import has_gpu
from .test_loader import real_corners

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def _rel(got, want):
    g, w = got.astype(np.float64), want.astype(np.float64)
    return np.abs(g - w).max() / np.abs(w).max()


@pytest.fixture(scope="module")
def moe_ckpt(tmp_path_factory):
    from escha_mlx_amd import loader
    path = tmp_path_factory.mktemp("moe")
    t = W.write_moe_checkpoint(path, np.random.default_rng(11), shards=2)
    return t, loader.load_model(path, device=DEV)


def _oracle_block_weights(t, i):
    p = W.PFX + f"layers.{i}.mlp."
    gu_code, dn_code = t[p + "experts.gate_up_proj.escha_code"], t[p + "experts.down_proj.escha_code"]
    E = gu_code.shape[0]
    w = {"gate_w": t[p + "gate.weight"], "shg_w": t[p + "shared_expert_gate.weight"],
         "gu": {"w": np.stack([R.reconstruct(gu_code[e], W.H, 2 * W.INTER, 2) for e in range(E)]),
                "rin": t[p + "experts.gate_up_proj.escha_rin"].astype(np.float32),
                "rout": t[p + "experts.gate_up_proj.escha_rout"].astype(np.float32)},
         "dn": {"w": np.stack([R.reconstruct(dn_code[e], W.INTER, W.H, 3) for e in range(E)]),
                "rin": t[p + "experts.down_proj.escha_rin"].astype(np.float32),
                "rout": t[p + "experts.down_proj.escha_rout"].astype(np.float32)}}
    for q in ("gate", "up", "down"):
        w[f"sh_{q}_w8"] = t[p + f"shared_expert.{q}_proj.weight_int8"]
        w[f"sh_{q}_scale"] = t[p + f"shared_expert.{q}_proj.weight_scale"]
    return w


@pytest.mark.parametrize("layer", [0, 1])
def test_loaded_moe_block_vs_oracle(moe_ckpt, layer):
    from escha_mlx_amd import moe, ops
    t, ck = moe_ckpt
    blk = ck[f"layers.{layer}.mlp"]
    rng = np.random.default_rng(20 + layer)
    x = rng.standard_normal((1, 3, W.H)).astype(np.float16)
    xd = torch.from_numpy(x).to(DEV)
    y = blk(xd)
    assert y.shape == (1, 3, W.H) and y.dtype == torch.float16
    got = y.cpu().numpy().reshape(3, W.H)
    w = _oracle_block_weights(t, layer)
    # the routing the block used, and the oracle's own routing of its logits
    logits = ops.gemv_f16w(xd.reshape(3, W.H), blk.gate_w).float()
    ids, scores = moe.route(logits, 2)
    o_ids, _ = R.route_topk(R.linear_f16(x.reshape(3, W.H), w["gate_w"]).astype(np.float32), 2)
    assert np.array_equal(np.sort(ids.cpu().numpy(), 1), np.sort(o_ids, 1))
    want = R.moe_block(x.reshape(3, W.H), w, 2, ids=ids.cpu().numpy(), scores=scores.cpu().numpy())
    assert _rel(got, want) < 5e-3
    assert torch.equal(blk(xd), y)
    # the int8 shared expert dominates the block's output here, so the routed
    # experts (the coded streams this layer loaded) are checked on their own
    routed = blk.experts(xd.reshape(3, W.H), ids, scores).cpu().numpy()
    want_r = R.moe_routed(x.reshape(3, W.H), ids.cpu().numpy(), scores.cpu().numpy(), w["gu"],
                          w["dn"], 2, 3, ordered=False)
    assert _rel(routed, want_r) < 5e-3


def test_loaded_embedding_and_last_position_head(moe_ckpt):
    from escha_mlx_amd import quant
    t, ck = moe_ckpt
    ids = np.array([[1, 2, 3, 4], [511, 0, 7, 7]])
    emb = ck["embed_tokens"](torch.from_numpy(ids).to(DEV))
    want = R.q8_embed(ids, t[W.PFX + "embed_tokens.weight_int8"], t[W.PFX + "embed_tokens.weight_scale"])
    assert np.array_equal(emb.cpu().numpy().view(np.uint16), want.view(np.uint16))
    head = ck["lm_head"]
    logits = head(emb)
    assert logits.shape == (2, 1, W.VOCAB)
    inner = head.inner
    assert isinstance(inner, quant.EschaQ8Head)
    assert torch.equal(logits, inner(emb[:, -1:, :]))
    ref = R.w8a16(want[:, -1, :], t["lm_head.weight_int8"], t["lm_head.weight_scale"])
    assert _rel(logits.cpu().numpy()[:, 0, :], ref) < 2e-3
    q = ck["layers.1.self_attn.q_proj"](emb[0])
    ref_q = R.w8a16(want[0], t[W.PFX + "layers.1.self_attn.q_proj.weight_int8"],
                    t[W.PFX + "layers.1.self_attn.q_proj.weight_scale"])
    assert _rel(q.cpu().numpy(), ref_q) < 2e-3


def test_loaded_dense_export_vs_deploy_and_oracle(tmp_path, monkeypatch):
    from escha_mlx_amd import loader
    monkeypatch.setenv("ESCHA_MLX_BIAS", "1")
    corners = real_corners()
    t = W.write_dense_checkpoint(tmp_path, np.random.default_rng(12), corners=corners)
    ck = loader.load_model(tmp_path, device=DEV)
    # the real corners: folded at load, bias applied, against the shipped output
    # (reference tests/test_dense_linear.py:68-78, REL_TOL 3e-3 on mean |diff|)
    for base, tag in W.REAL_CORNERS.items():
        g = corners[tag]
        y = ck[base](torch.from_numpy(g["x"]).to(DEV)).cpu().numpy().astype(np.float32)
        dep = g["deploy"].astype(np.float32)
        assert np.abs(y - dep).mean() / np.abs(dep).mean() < 3e-3, base
        rin, rout = R.fold_scales(g["rin"], g["rout"], g["s_in"], g["s_out"])
        want = R.dense_linear(g["x"], g["code"], rin, rout, g["K"], bias=g["bias"])
        assert _rel(y, want) < 2e-3, base
    # every synthetic projection at 1 and 4 rows against the oracle
    rng = np.random.default_rng(13)
    for base, (ic, oc, K) in W.DENSE_PROJ.items():
        p = W.PFX + base
        rin, rout = R.fold_scales(t[p + ".escha_rin"], t[p + ".escha_rout"], t[p + ".escha_s_in"],
                                  t[p + ".escha_s_out"])
        for m in (1, 4):
            x = rng.standard_normal((m, ic)).astype(np.float16)
            y = ck[base](torch.from_numpy(x).to(DEV)).cpu().numpy()
            want = R.dense_linear(x, t[p + ".escha_code"], rin, rout, K, bias=t[p + ".bias"])
            assert _rel(y, want) < 2e-3, (base, m)
