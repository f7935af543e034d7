"""GPU parity of esc_linear, the whole coded linear in one call
(EschaLinear.__call__, escha_mlx/dense.py:337-362).

Exactness is checked where the float32 sum has a single term: with
x = rin * H128[:, k] (one Sylvester column) the input transform gives exactly
f16(128 * RS) at input k and zeros elsewhere, so the output must equal the
oracle's output transform of f16(128 RS) * W[k] bit-for-bit (decode, lane
layout, split-K bookkeeping, output transform and bias all pinned).  Random
inputs are held to the float16 tolerance of the split-K GEMV against a float64
product, and repeated calls on one workspace must be bit-identical (its
counters reset themselves).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu

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


def _proj(rng, ic, oc, K):
    u32 = rng.integers(0, 2**32, size=(ic // 16, oc // 16, 8 * K), dtype=np.uint64).astype(np.uint32)
    rin = rng.choice([-1.0, 1.0], ic).astype(np.float32)
    rout = (rng.choice([-1.0, 1.0], oc) * rng.uniform(0.5, 1.5, oc) * 1e-2).astype(np.float32)
    return u32, rin, rout


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _code(u32):
    return _dev(u32.view(np.int32))


def _sylvester128():
    h = np.array([[1.0]])
    for _ in range(7):
        h = np.block([[h, h], [h, -h]])
    return h


# 9..15 rows: (2, 1024, 1024, 9), (3, 2048, 384, 13) and (2, 5120, 5120, 15)
# run as two row groups (one group at its fewest splits would leave the GPU
# short of workgroups), (3, 4096, 8192, 12) as one group of 12 rows
@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,ic,oc,m", [(2, 2048, 2048, 1), (2, 5120, 640, 3), (3, 1024, 1152, 7),
                                       (3, 2048, 384, 13), (2, 1024, 1024, 9), (2, 5120, 5120, 4),
                                       (2, 5120, 5120, 15), (3, 4096, 8192, 12)])
def test_linear_single_term_bit_exact(K, ic, oc, m, lut):
    rng = np.random.default_rng(100 * K + m)
    u32, rin, rout = _proj(rng, ic, oc, K)
    bias = (rng.standard_normal(oc) * 0.05).astype(np.float16)
    hs = _sylvester128()
    ks = rng.integers(0, ic, size=m)
    x = np.zeros((m, ic), np.float32)
    for r, k in enumerate(ks):
        blk = 128 * (k // 128)
        x[r, blk:blk + 128] = hs[:, k % 128] * rin[blk:blk + 128]
    x16 = x.astype(np.float16)
    y = ops().linear(_dev(x16), _code(u32), _dev(rin), _dev(rout), K, ic, oc, bias=_dev(bias),
                     lut=lut).cpu().numpy()
    xh = R.input_transform(x16, rin)
    w = R.reconstruct(u32, ic, oc, K)
    for r, k in enumerate(ks):
        assert np.count_nonzero(xh[r]) == 1 and xh[r, k] != 0
        mid = (xh[r, k].astype(np.float32) * w[k].astype(np.float32))[None]
        want = R.output_transform(mid, rout)[0]
        want = (want.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
        assert np.array_equal(y[r].view(np.uint16), want.view(np.uint16)), r


@pytest.mark.parametrize("K,ic,oc,m,lut", [(2, 5120, 1024, 1, True), (2, 5120, 5120, 1, True),
                                           (3, 5120, 2048, 4, True), (3, 5120, 2048, 4, False),
                                           (3, 17408 // 4, 640, 2, False), (2, 2048, 2048, 15, False),
                                           (2, 1024, 768, 40, False)])
def test_linear_vs_f64_and_repeatable(K, ic, oc, m, lut):
    rng = np.random.default_rng(7 * K + m)
    u32, rin, rout = _proj(rng, ic, oc, K)
    x = rng.standard_normal((m, ic)).astype(np.float16)
    ws = torch.zeros(max(ops().linear_workspace(m, K, ic, oc), 4), dtype=torch.uint8, device=DEV)
    args = (_dev(x), _code(u32), _dev(rin), _dev(rout), K, ic, oc)
    y = ops().linear(*args, lut=lut, ws=ws)
    xh = R.input_transform(x, rin)
    w = R.reconstruct(u32, ic, oc, K)
    exact = R.h128(R.gemv_f64(xh, w).astype(np.float32)) * R.RS * rout
    got = y.cpu().numpy().astype(np.float32)
    err = (np.abs(got - exact).max(axis=1) / np.abs(exact).max(axis=1)).max()
    assert err < 2e-3, err
    for _ in range(3):
        assert torch.equal(ops().linear(*args, lut=lut, ws=ws), y)


def test_linear_workspace_shared_by_table_and_hash_calls():
    """Table and hash calls on one workspace (different split plans) stay
    bit-identical to each other: the counters sit where both plans expect."""
    rng = np.random.default_rng(11)
    K, ic, oc = 2, 5120, 5120
    u32, rin, rout = _proj(rng, ic, oc, K)
    x = rng.standard_normal((1, ic)).astype(np.float16)
    ws = torch.zeros(max(ops().linear_workspace(1, K, ic, oc), 4), dtype=torch.uint8, device=DEV)
    args = (_dev(x), _code(u32), _dev(rin), _dev(rout), K, ic, oc)
    first = {lut: ops().linear(*args, lut=lut, ws=ws) for lut in (True, False)}
    for _ in range(3):
        for lut in (True, False, True):
            assert torch.equal(ops().linear(*args, lut=lut, ws=ws), first[lut]), lut


def test_linear_workspace_shared_two_row_groups():
    """9-15 rows: the workspace's counters are sized for two row groups per
    column group (the hash plan here splits 12 rows into two groups of 6:
    48 column groups x 5 splits < 256 workgroups).  A request for the table
    decode runs the same hash plan (the two decodes give the same weights), so
    alternating requests on one workspace give the same bits."""
    rng = np.random.default_rng(12)
    K, ic, oc, m = 2, 5120, 12288, 12
    u32, rin, rout = _proj(rng, ic, oc, K)
    x = rng.standard_normal((m, ic)).astype(np.float16)
    ws = torch.zeros(max(ops().linear_workspace(m, K, ic, oc), 4), dtype=torch.uint8, device=DEV)
    args = (_dev(x), _code(u32), _dev(rin), _dev(rout), K, ic, oc)
    fresh = {lut: ops().linear(*args, lut=lut, ws=torch.zeros_like(ws)) for lut in (True, False)}
    assert torch.equal(fresh[True], fresh[False])
    for _ in range(3):
        for lut in (False, True, False, True):
            assert torch.equal(ops().linear(*args, lut=lut, ws=ws), fresh[lut]), lut


def test_module_default_uses_one_launch_linear(monkeypatch):
    """EschaLinear below 16 rows defaults to esc_linear; within tolerance of the
    order-exact module (ESCHA_HIP_EXACT=1), bias included."""
    from escha_mlx_amd.dense import EschaLinear, EschaWeight
    rng = np.random.default_rng(5)
    ic, oc, K = 1024, 768, 2
    code = rng.integers(-32768, 32768, size=(ic // 16, oc // 16, 16 * K), dtype=np.int16)
    rin = rng.choice([-1.0, 1.0], ic).astype(np.float16)
    rout = (rng.choice([-1.0, 1.0], oc) * rng.uniform(0.5, 1.5, oc) * 1e-2).astype(np.float16)
    bias = (rng.standard_normal(oc) * 0.05).astype(np.float16)
    w = EschaWeight(code, rin, rout, device=DEV)
    for m in (1, 6):
        x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
        monkeypatch.delenv("ESCHA_HIP_EXACT", raising=False)
        y_fast = EschaLinear(w, bias=bias)(x).float()
        monkeypatch.setenv("ESCHA_HIP_EXACT", "1")
        y_exact = EschaLinear(w, bias=bias)(x).float()
        assert float((y_fast - y_exact).abs().max() / y_exact.abs().max()) < 2e-3


@pytest.mark.parametrize("K,ic,oc,m", [(2, 1024, 1024, 40), (3, 512, 2048, 300), (2, 256, 4096, 600),
                                       (3, 1024, 768, 33), (2, 512, 640, 50)])
def test_linear_many_rows_fused_epilogue_equals_three_launches(K, ic, oc, m):
    """From 16 rows esc_linear runs the input transform and the matrix-core GEMM
    with the output transform in its epilogue (OC a multiple of 256; otherwise
    GEMM + output transform): bit-identical to the three separate C-ABI calls."""
    rng = np.random.default_rng(3 * K + m)
    u32, rin, rout = _proj(rng, ic, oc, K)
    bias = _dev((rng.standard_normal(oc) * 0.05).astype(np.float16))
    x = _dev(rng.standard_normal((m, ic)).astype(np.float16))
    code, rin_d, rout_d = _code(u32), _dev(rin), _dev(rout)
    for b in (None, bias):
        y = ops().linear(x, code, rin_d, rout_d, K, ic, oc, bias=b)
        xh = ops().scaled_had(x, rin_d, None)
        mid = ops().dense_gemm_mat(xh, code, K, ic, oc)
        want = ops().scaled_had_out(mid, rout_d, None, bias=b)
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
