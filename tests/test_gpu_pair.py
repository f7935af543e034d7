"""GPU parity of the projection-pair dispatch (dense.project_pair,
escha_mlx/dense.py:365-437) and the modules built on it (the fused MLP and the
k/v pair of escha_mlx/models/qwen3_5.py:63-198).

The pair launch runs each projection's own one-launch plan, so its outputs
must equal two separate esc_linear calls bit for bit, for every rate
combination, both decode modes and every row count; the fused MLP is held to
the oracle's linear -> SwiGLU -> linear chain.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu
from .test_gpu_linear import _code, _dev, _proj

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


def _p(rng, ic, oc, K, bias):
    u32, rin, rout = _proj(rng, ic, oc, K)
    b = _dev((rng.standard_normal(oc) * 0.01).astype(np.float16)) if bias else None
    return (_code(u32), _dev(rin), _dev(rout), K, oc, b)


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K0,K1", [(2, 2), (2, 3), (3, 2), (3, 3)])
@pytest.mark.parametrize("m", [1, 4, 15, 16, 24])
def test_pair_bit_identical_to_single_linears(K0, K1, m, lut):
    rng = np.random.default_rng(100 * K0 + 10 * K1 + m)
    ic = 1024
    p0 = _p(rng, ic, 384, K0, True)    # 24 tiles: a partial K=2 column group
    p1 = _p(rng, ic, 1280, K1, False)
    x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
    o = ops()
    y0, y1 = o.linear_pair(x, p0, p1, lut=lut)
    s0 = o.linear(x, p0[0], p0[1], p0[2], K0, ic, p0[4], bias=p0[5], lut=lut)
    s1 = o.linear(x, p1[0], p1[1], p1[2], K1, ic, p1[4], bias=p1[5], lut=lut)
    assert torch.equal(y0, s0) and torch.equal(y1, s1)
    # one workspace reused: the counters reset themselves
    ws = torch.zeros(o.linear_pair_workspace(m, K0, K1, ic, 384, 1280), dtype=torch.uint8, device=DEV)
    for _ in range(2):
        z0, z1 = o.linear_pair(x, p0, p1, lut=lut, ws=ws)
        assert torch.equal(z0, s0) and torch.equal(z1, s1)


def test_pair_with_different_row_groups_is_two_linears():
    """12 rows: projection 0 (24 tiles) runs as two row groups of 6, projection
    1 (K=3, 4096 -> 8192: 64 column groups x 4 splits fill 256 workgroups) as
    one group of 12; the pair then runs each projection's own call, bit for
    bit."""
    rng = np.random.default_rng(4242)
    ic, m = 4096, 12
    p0 = _p(rng, ic, 384, 2, True)
    p1 = _p(rng, ic, 8192, 3, False)
    x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
    o = ops()
    s0 = o.linear(x, p0[0], p0[1], p0[2], 2, ic, 384, bias=p0[5])
    s1 = o.linear(x, p1[0], p1[1], p1[2], 3, ic, 8192, bias=p1[5])
    ws = torch.zeros(o.linear_pair_workspace(m, 2, 3, ic, 384, 8192), dtype=torch.uint8, device=DEV)
    for _ in range(2):
        y0, y1 = o.linear_pair(x, p0, p1, ws=ws)
        assert torch.equal(y0, s0) and torch.equal(y1, s1)


@pytest.mark.parametrize("K", [2, 3])
@pytest.mark.parametrize("m", [2, 4, 15, 16, 24])
def test_multi_rows_bit_identical_to_single_linears(K, m):
    """esc_linear_multi at several rows: q, k and v style projections of one
    input in one k_linear_multi launch (below 16 rows) or one call each, every
    output bit-identical to its own esc_linear call; a reused workspace keeps
    giving the same bits."""
    rng = np.random.default_rng(500 + 10 * K + m)
    ic = 1024
    projs = [_p(rng, ic, 384, K, True), _p(rng, ic, 1280, K, False), _p(rng, ic, 512, K, True)]
    x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
    o = ops()
    want = [o.linear(x, p[0], p[1], p[2], K, ic, p[4], bias=p[5]) for p in projs]
    ys = o.linear_multi(x, projs)
    assert all(torch.equal(y, w) for y, w in zip(ys, want))
    ws = torch.zeros(o.linear_multi_workspace(K, ic, [p[4] for p in projs], m), dtype=torch.uint8,
                     device=DEV)
    for _ in range(2):
        ys = o.linear_multi(x, projs, lut=True, ws=ws)
        assert all(torch.equal(y, w) for y, w in zip(ys, want))


def test_multi_rows_with_different_row_groups_is_separate_linears():
    """12 rows, K=3: projection 0 (3 column groups) runs as two row groups of
    6, projection 1 (4096 -> 8192: 64 column groups x 4 splits) as one group
    of 12, so the call runs each projection's own esc_linear, bit for bit."""
    rng = np.random.default_rng(4343)
    ic, m = 4096, 12
    projs = [_p(rng, ic, 384, 3, True), _p(rng, ic, 8192, 3, False)]
    x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
    o = ops()
    want = [o.linear(x, p[0], p[1], p[2], 3, ic, p[4], bias=p[5]) for p in projs]
    ys = o.linear_multi(x, projs)
    assert all(torch.equal(y, w) for y, w in zip(ys, want))


def _linear_mod(rng, ic, oc, K, bias=None):
    from escha_mlx_amd import dense
    u32, rin, rout = _proj(rng, ic, oc, K)
    code_i16 = u32.view(np.int16).reshape(ic // 16, oc // 16, 16 * K)
    g = {"escha_code": code_i16, "escha_rin": rin, "escha_rout": rout}
    if bias is not None:
        g["bias"] = bias
    return dense.build(g, device=DEV), (code_i16, rin, rout)


@pytest.mark.parametrize("m", [1, 3, 20])
def test_project_pair_and_fused_mlp_vs_oracle(m):
    from escha_mlx_amd import dense
    rng = np.random.default_rng(7 + m)
    H, I = 512, 384
    gate, (gc, gri, gro) = _linear_mod(rng, H, I, 2)
    up, (uc, uri, uro) = _linear_mod(rng, H, I, 3)
    down, (dc, dri, dro) = _linear_mod(rng, I, H, 3)
    x = rng.standard_normal((m, H)).astype(np.float16)
    xd = _dev(x)
    g, u = dense.project_pair(gate, up, xd)
    assert torch.equal(g, gate(xd)) and torch.equal(u, up(xd))
    mlp = dense.EschaMLP(gate, up, down)
    y = mlp(xd).cpu().numpy()
    g_o = R.dense_linear(x, gc, gri, gro, 2)
    u_o = R.dense_linear(x, uc, uri, uro, 3)
    h_o = R.shared_act(g_o, u_o)
    want = R.dense_linear(h_o, dc, dri, dro, 3)
    assert np.abs(y.astype(np.float64) - want).max() / np.abs(want).max() < 5e-3
    # the module's own activation is the oracle's on the module's gate / up
    h = ops().moe_shared_act(g, u).cpu().numpy()
    ulps = np.abs(h.view(np.int16).astype(np.int32) - R.shared_act(g.cpu().numpy(), u.cpu().numpy())
                  .view(np.int16).astype(np.int32))
    assert ulps.max() <= 1


@pytest.mark.parametrize("m", [1, 3])
def test_project_many_vs_oracle(m):
    """q, k and v of one input in one launch: at one row within the float16
    tolerance of the oracle's projections, at 3 rows also bit-identical to
    each module's own call."""
    from escha_mlx_amd import dense
    rng = np.random.default_rng(11 + m)
    IC = 1024
    mods = [_linear_mod(rng, IC, oc, 2, bias=(rng.standard_normal(oc) * 0.02).astype(np.float16)
                        if oc == 512 else None) for oc in (512, 256, 768)]
    x = rng.standard_normal((m, IC)).astype(np.float16)
    xd = _dev(x)
    ys = dense.project_many([mm for mm, _ in mods], xd)
    for (mod, (code, rin, rout)), y in zip(mods, ys):
        want = R.dense_linear(x, code, rin, rout, 2)
        if mod.bias is not None:
            want = (want.astype(np.float32) + mod.bias.cpu().numpy().astype(np.float32))
        got = y.cpu().numpy().astype(np.float64)
        assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
        if m > 1:
            assert torch.equal(y, mod(xd))


def test_project_pair_falls_back_when_incompatible(monkeypatch):
    from escha_mlx_amd import dense
    rng = np.random.default_rng(3)
    a, _ = _linear_mod(rng, 512, 256, 2)
    b, _ = _linear_mod(rng, 1024, 256, 2)   # another input width
    x = _dev(rng.standard_normal((2, 512)).astype(np.float16))
    with pytest.raises(ValueError):
        dense.project_pair(a, b, x)           # b(x) itself rejects the width
    monkeypatch.setenv("ESCHA_HIP_EXACT", "1")
    c, _ = _linear_mod(rng, 512, 256, 3)     # order-exact module: two calls
    y0, y1 = dense.project_pair(a, c, x)
    assert torch.equal(y0, a(x)) and torch.equal(y1, c(x))


def test_loader_installs_fused_mlp_and_kv(tmp_path, monkeypatch):
    from escha_mlx_amd import dense, loader

    from . import ckpt_writer as W
    monkeypatch.setenv("ESCHA_MLX_BIAS", "1")
    W.write_dense_checkpoint(tmp_path, np.random.default_rng(21))
    ck = loader.load_model(tmp_path, device=DEV)
    mlp = ck["layers.0.mlp"]
    assert isinstance(mlp, dense.EschaMLP)
    kv = ck["layers.1.self_attn.kv"]
    x = _dev(np.random.default_rng(5).standard_normal((1, 2, W.H)).astype(np.float16))
    k, v = kv(x)
    assert torch.equal(k, ck["layers.1.self_attn.k_proj"](x))
    assert torch.equal(v, ck["layers.1.self_attn.v_proj"](x))
    y = mlp(x)
    assert y.shape == (1, 2, W.H)
    assert torch.equal(y, ck["layers.0.mlp.down_proj"](
        ops().moe_shared_act(ck["layers.0.mlp.gate_proj"](x).reshape(2, -1).contiguous(),
                             ck["layers.0.mlp.up_proj"](x).reshape(2, -1).contiguous())
    ).reshape(1, 2, W.H))
