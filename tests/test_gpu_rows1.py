"""GPU parity of the one-row persistent projection kernel (k_proj_rows1):
esc_linear_multi (one to four projections of one row; one projection is
exactly esc_linear's computation), and esc_linear / esc_linear_pair at M = 1
where they take it (table decode, at least 16,384 kt x 256-column units;
smaller projections run the split-K kernel by hash whichever decode is asked
for) (EschaLinear.__call__, escha_mlx/dense.py:337-362).

Shapes are chosen to exercise the kernel's bookkeeping: one unit per wave
(small projections), ranges that cross a 128-input block and a column group,
column groups spread over many workgroups (IC = 17408 / 4, 5120), and a
single column group.  Exactness: with x = rin * H128[:, k] the input transform
leaves one non-zero input, so every output equals the oracle's output
transform of f16(128 RS) * W[k] bit-for-bit (decode, lane and column
layout, partial bookkeeping, output transform and bias pinned).  Random
inputs: within the float16 tolerance of a float64 product, bit-identical on
repeated calls over one workspace, and a pair launch bit-identical to the two
single launches.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu
from .test_gpu_linear import _code, _dev, _proj, _sylvester128

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


SHAPES = [(2, 128, 256), (2, 1024, 4096), (2, 5120, 1280), (2, 4352, 512), (3, 128, 512),
          (3, 2048, 1024), (3, 4352, 768), (3, 1024, 2816), (2, 8192, 3072), (2, 8192, 8192)]


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,ic,oc", SHAPES)
def test_rows1_single_term_bit_exact(K, ic, oc, lut):
    rng = np.random.default_rng(ic + oc + K)
    u32, rin, rout = _proj(rng, ic, oc, K)
    bias = (rng.standard_normal(oc) * 0.05).astype(np.float16)
    hs = _sylvester128()
    w = R.reconstruct(u32, ic, oc, K)
    for k in (0, ic - 1, int(rng.integers(0, ic))):
        blk = 128 * (k // 128)
        x = np.zeros((1, ic), np.float32)
        x[0, blk:blk + 128] = hs[:, k % 128] * rin[blk:blk + 128]
        x16 = x.astype(np.float16)
        y = ops().linear_multi(_dev(x16), [(_code(u32), _dev(rin), _dev(rout), K, oc, _dev(bias))],
                               lut=lut)[0].cpu().numpy()
        xh = R.input_transform(x16, rin)
        assert np.count_nonzero(xh[0]) == 1 and xh[0, k] != 0
        mid = (xh[0, k].astype(np.float32) * w[k].astype(np.float32))[None]
        want = R.output_transform(mid, rout)[0]
        want = (want.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
        assert np.array_equal(y[0].view(np.uint16), want.view(np.uint16)), k


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,ic,oc", SHAPES)
def test_rows1_vs_f64_and_repeatable(K, ic, oc, lut):
    rng = np.random.default_rng(3 * ic + oc + K)
    u32, rin, rout = _proj(rng, ic, oc, K)
    x = rng.standard_normal((1, ic)).astype(np.float16)
    ws = torch.zeros(ops().linear_multi_workspace(K, ic, [oc]), dtype=torch.uint8, device=DEV)
    proj = [(_code(u32), _dev(rin), _dev(rout), K, oc, None)]
    run = lambda lt: ops().linear_multi(_dev(x), proj, lut=lt, ws=ws)[0]
    y = run(lut)
    xh = R.input_transform(x, rin)
    w = R.reconstruct(u32, ic, oc, K)
    exact = R.h128(R.gemv_f64(xh, w).astype(np.float32)) * R.RS * rout
    got = y.cpu().numpy().astype(np.float32)
    err = np.abs(got - exact).max() / np.abs(exact).max()
    assert err < 2e-3, err
    for _ in range(3):
        assert torch.equal(run(lut), y)
    # the other decode on the same workspace: the same weights, the same plan
    assert torch.equal(run(not lut), y)
    # esc_linear on the same row: the same computation where it takes this
    # kernel, within the tolerance contract where it takes the split-K one
    single = ops().linear(_dev(x), _code(u32), _dev(rin), _dev(rout), K, ic, oc, lut=lut)
    if lut and (ic // 16) * (oc // 256) >= 16384:
        assert torch.equal(single, y)
    s32 = single.cpu().numpy().astype(np.float32)
    assert np.abs(s32 - exact).max() / np.abs(exact).max() < 2e-3


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,ic,oc0,oc1", [(2, 1024, 256, 1280), (3, 2048, 768, 512),
                                          (2, 8192, 3072, 3072), (3, 6144, 4096, 4096),
                                          (2, 8192, 3072, 512), (2, 8192, 8192, 8192),
                                          (2, 8192, 8192, 3072)])
def test_rows1_pair_bit_identical_to_single(K, ic, oc0, oc1, lut):
    rng = np.random.default_rng(ic + oc0 + 7 * oc1)
    o = ops()
    ps = []
    for oc, with_bias in ((oc0, True), (oc1, False)):
        u32, rin, rout = _proj(rng, ic, oc, K)
        b = _dev((rng.standard_normal(oc) * 0.01).astype(np.float16)) if with_bias else None
        ps.append((_code(u32), _dev(rin), _dev(rout), K, oc, b))
    x = _dev(rng.standard_normal((1, ic)).astype(np.float16))
    s0 = o.linear(x, ps[0][0], ps[0][1], ps[0][2], K, ic, oc0, bias=ps[0][5], lut=lut)
    s1 = o.linear(x, ps[1][0], ps[1][1], ps[1][2], K, ic, oc1, bias=ps[1][5], lut=lut)
    ws = torch.zeros(o.linear_pair_workspace(1, K, K, ic, oc0, oc1), dtype=torch.uint8, device=DEV)
    for _ in range(3):
        y0, y1 = o.linear_pair(x, ps[0], ps[1], lut=lut, ws=ws)
        assert torch.equal(y0, s0) and torch.equal(y1, s1)


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,ic,ocs", [(2, 5120, (5120, 1024, 1024)), (3, 1024, (512, 2816)),
                                      (2, 128, (256, 256, 512, 768)), (3, 2048, (256,))])
def test_rows1_multi_projections(K, ic, ocs, lut):
    """esc_linear_multi: several projections of one row in one launch (a
    shared plan).  Single-term inputs give every output bit-exact; random
    inputs are within the float16 tolerance of float64 products and repeated
    calls on one workspace are bit-identical."""
    rng = np.random.default_rng(ic + sum(ocs) + K)
    o = ops()
    projs, host = [], []
    for i, oc in enumerate(ocs):
        u32, rin, rout = _proj(rng, ic, oc, K)
        b = (rng.standard_normal(oc) * 0.02).astype(np.float16) if i % 2 == 0 else None
        projs.append((_code(u32), _dev(rin), _dev(rout), K, oc, None if b is None else _dev(b)))
        host.append((R.reconstruct(u32, ic, oc, K), rin, rout, b))
    hs = _sylvester128()
    k = int(rng.integers(0, ic))
    blk = 128 * (k // 128)
    # x is shared: the Sylvester column scaled by the first projection's rin
    # leaves one input only for projections with the same signs, so each
    # projection gets its own single-term row in turn
    for j in range(len(ocs)):
        x = np.zeros((1, ic), np.float32)
        x[0, blk:blk + 128] = hs[:, k % 128] * host[j][1][blk:blk + 128]
        x16 = x.astype(np.float16)
        ys = o.linear_multi(_dev(x16), projs, lut=lut)
        w, rin, rout, b = host[j]
        xh = R.input_transform(x16, rin)
        assert np.count_nonzero(xh[0]) == 1
        want = R.output_transform((xh[0, k].astype(np.float32) * w[k].astype(np.float32))[None], rout)[0]
        if b is not None:
            want = (want.astype(np.float32) + b.astype(np.float32)).astype(np.float16)
        assert np.array_equal(ys[j].cpu().numpy()[0].view(np.uint16), want.view(np.uint16)), j
    x16 = rng.standard_normal((1, ic)).astype(np.float16)
    ws = torch.zeros(o.linear_multi_workspace(K, ic, list(ocs)), dtype=torch.uint8, device=DEV)
    ys = o.linear_multi(_dev(x16), projs, lut=lut, ws=ws)
    for (w, rin, rout, b), y in zip(host, ys):
        xh = R.input_transform(x16, rin)
        exact = R.h128(R.gemv_f64(xh, w).astype(np.float32)) * R.RS * rout
        if b is not None:
            exact = exact + b.astype(np.float32)
        got = y.cpu().numpy().astype(np.float32)
        assert np.abs(got - exact).max() / np.abs(exact).max() < 2e-3
    for _ in range(2):
        again = o.linear_multi(_dev(x16), projs, lut=lut, ws=ws)
        assert all(torch.equal(a, b) for a, b in zip(again, ys))
