"""GPU parity of the dense int8 / f16 GEMV and the whole MoE block
(escha_mlx/quant.py w8a16 contract, models/qwen3_5_moe.py:257-273,
ref.moe_block escha_mlx/ref.py:314-349), through the C-ABI.

One-hot inputs pin every weight bit-exactly (a single product: x = e_k makes
y[:, o] the contract weight f16(f32(w8[o, k]) * f32(scale[o]))); other inputs
are held to the reference's own w8a16 bar (max |diff| / max |want| < 2e-3,
tests/test_mlx_cpu.py:55-65 of the reference) against its golden and against
a float64 product of the contract weights.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu, moe_block_weights

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def ops():
    from escha_mlx_amd import ops as o
    return o


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _rel(got, want):
    g, w = got.astype(np.float64), want.astype(np.float64)
    return np.abs(g - w).max() / np.abs(w).max()


def test_w8a16_vs_reference_golden(w8a16_golden):
    w8, scale, x, want = w8a16_golden
    got = ops().w8a16(_dev(x), _dev(w8), _dev(scale)).cpu().numpy()
    assert _rel(got, want) < 2e-3
    wf = (w8.astype(np.float32) * scale[:, None]).astype(np.float16).astype(np.float64)
    assert _rel(got, x.astype(np.float64) @ wf.T) < 2e-3


# K = 128 / 256 / 384: 8 / 16 / 32 lanes per row (384: 24 chunks, 8 lanes
# idle); 5120 and 8192: 5 and 8 chunks per lane, at most 2 rows per launch
@pytest.mark.parametrize("K", [128, 256, 384, 512, 1024, 2048, 4096, 5120, 8192])
@pytest.mark.parametrize("m", [1, 3, 8, 11])
def test_w8a16_one_hot_bit_exact(K, m):
    rng = np.random.default_rng(K + m)
    O = (384 if K < 4096 else 96) + 1  # a partial last wave-step where rows share a wave
    w8 = rng.integers(-128, 128, size=(O, K), dtype=np.int8)
    scale = rng.uniform(1e-3, 5e-3, O).astype(np.float16).astype(np.float32)
    ks = rng.integers(0, K, size=m)
    x = np.zeros((m, K), np.float16)
    x[np.arange(m), ks] = 1.0
    got = ops().w8a16(_dev(x), _dev(w8), _dev(scale)).cpu().numpy()
    for r, k in enumerate(ks):
        want = (w8[:, k].astype(np.float32) * scale).astype(np.float16)
        assert np.array_equal(got[r].view(np.uint16), want.view(np.uint16)), r


@pytest.mark.parametrize("K,m", [(2048, 1), (512, 4), (1024, 8), (2048, 13), (256, 3), (384, 9),
                                 (5120, 5), (8192, 3)])
def test_w8a16_vs_f64_and_deterministic(K, m):
    rng = np.random.default_rng(3 * K + m)
    O = 640
    w8 = rng.integers(-128, 128, size=(O, K), dtype=np.int8)
    scale = rng.uniform(1e-3, 5e-3, O).astype(np.float32)
    x = rng.standard_normal((m, K)).astype(np.float16)
    args = (_dev(x), _dev(w8), _dev(scale))
    y = ops().w8a16(*args)
    wf = (w8.astype(np.float32) * scale[:, None]).astype(np.float16).astype(np.float64)
    assert _rel(y.cpu().numpy(), x.astype(np.float64) @ wf.T) < 2e-3
    assert torch.equal(ops().w8a16(*args), y)


@pytest.mark.parametrize("K", [64, 200, 256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("m", [1, 5, 9])
def test_gemv_f16w_one_hot_and_f64(K, m):
    rng = np.random.default_rng(7 * K + m)
    O = 256
    w = (rng.standard_normal((O, K)) * 0.05).astype(np.float16)
    ks = rng.integers(0, K, size=m)
    x = np.zeros((m, K), np.float16)
    x[np.arange(m), ks] = 1.0
    got = ops().gemv_f16w(_dev(x), _dev(w)).cpu().numpy()
    for r, k in enumerate(ks):
        assert np.array_equal(got[r].view(np.uint16), w[:, k].view(np.uint16))
    xr = rng.standard_normal((m, K)).astype(np.float16)
    got = ops().gemv_f16w(_dev(xr), _dev(w)).cpu().numpy()
    assert _rel(got, xr.astype(np.float64) @ w.astype(np.float64).T) < 2e-3


def test_shared_act_and_block_out_vs_oracle():
    rng = np.random.default_rng(9)
    g = (rng.standard_normal((5, 512)) * 3).astype(np.float16)
    u = rng.standard_normal((5, 512)).astype(np.float16)
    got = ops().moe_shared_act(_dev(g), _dev(u)).cpu().numpy()
    want = R.shared_act(g, u)
    # device expf vs numpy exp: at most one f16 ulp apart
    ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01
    y = rng.standard_normal((5, 512)).astype(np.float16)
    sh = rng.standard_normal((5, 512)).astype(np.float16)
    shg = (rng.standard_normal((5, 1)) * 2).astype(np.float16)
    got = ops().moe_block_out(_dev(y), _dev(sh), _dev(shg)).cpu().numpy()
    sg = np.float32(1) / (np.float32(1) + np.exp(-shg.astype(np.float32)))
    want = (y.astype(np.float32) + sh.astype(np.float32) * sg).astype(np.float16)
    ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1


def _block(v):
    from escha_mlx_amd import moe
    E, H = v["blk_gate_w"].shape
    gu = moe.EschaExperts(v["blk_gu_code"], v["blk_gu_rin"], v["blk_gu_rout"], device=DEV)
    dn = moe.EschaExperts(v["blk_dn_code"], v["blk_dn_rin"], v["blk_dn_rout"], device=DEV)
    shared = {f"{p}_{leaf}": v[f"blk_sh_{p}_{leaf}"] for p in ("gate", "up", "down")
              for leaf in ("w8", "scale")}
    return moe.EschaSparseMoeBlock(H, E, 2, gu, dn, v["blk_gate_w"], v["blk_shg_w"], shared)


def test_moe_block_vs_oracle_and_reference(ref_vectors):
    """The whole block against the oracle (same rounding points) and against
    ref.moe_block's own output (which keeps the routed sum in float64)."""
    v = ref_vectors
    blk = _block(v)
    x = _dev(v["blk_x"])
    y = blk(x)
    got = y.cpu().numpy()
    want = R.moe_block(v["blk_x"], moe_block_weights(v), 2)
    assert _rel(got, want) < 5e-3
    assert _rel(got, v["blk_y"]) < 5e-3
    assert torch.equal(blk(x), y)


@pytest.mark.parametrize("K", [256, 2048])
def test_q8_embed_bit_exact(K):
    """Embedding rows are the contract weights, bit for bit (the same rounding
    the w8a16 golden pins); an id outside the table gives a NaN row."""
    from escha_mlx_amd import quant
    rng = np.random.default_rng(K)
    N = 300
    w8 = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    scale = rng.uniform(1e-3, 5e-3, N).astype(np.float16)  # f16 scales, as exported
    emb = quant.make_embedding(w8, scale, device=DEV)
    ids = rng.integers(0, N, size=(2, 5))
    got = emb(torch.from_numpy(ids).to(DEV))
    assert got.shape == (2, 5, K) and got.dtype == torch.float16
    want = R.q8_embed(ids, w8, scale)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))
    bad = emb(torch.tensor([0, N, -1, N - 1], device=DEV)).cpu().numpy()
    assert np.isnan(bad[1]).all() and np.isnan(bad[2]).all()
    assert np.array_equal(bad[[0, 3]].view(np.uint16), R.q8_embed(np.array([0, N - 1]), w8, scale).view(np.uint16))
