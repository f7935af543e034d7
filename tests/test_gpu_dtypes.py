"""bf16 and f32 activations, as the reference takes them: the rows are
transformed from their exact float32 values with no f16 rounding first
(EschaLinear._input_rows, escha_mlx/dense.py:287-292; the expert path's
_scaled_had, escha_mlx/models/qwen3_5_moe.py:103-110), and the module output
is cast back to the input's dtype (dense.py:362).

The oracle's input transform reads float32 rows, so bf16 rows are held as
float32 arrays of bf16-representable values (the low 16 bits of each float32
cleared) and float32 rows as they are.  The transform is then bit-exact; the
order-exact modules (ESCHA_HIP_EXACT=1) are bit-exact end to end, the default
modules within the float16 tolerance of a float64 product.  A float32 row
whose f16 rounding changes the result shows that no f16 rounding happened.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu
from .test_gpu_parity import _block, _moe_case, _oracle_moe, bits16

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


def _rows(rng, shape, dtype):
    """(host float32 values, device tensor of `dtype` holding exactly them)."""
    v = (rng.standard_normal(shape) * 3.0).astype(np.float32)
    if dtype == torch.bfloat16:
        v = (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    t = torch.from_numpy(v).to(DEV).to(dtype)
    assert np.array_equal(t.float().cpu().numpy().view(np.uint32), v.view(np.uint32))
    return v, t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("m,IC,E", [(5, 512, 1), (33, 1024, 7)])
def test_input_transform_typed_bit_exact(dtype, m, IC, E):
    rng = np.random.default_rng(m + IC + E)
    v, x = _rows(rng, (m, IC), dtype)
    if E == 1:
        rin = rng.choice([-1.0, 1.0], IC).astype(np.float32) * np.float32(0.75)
        re, re_np, rin_rows = None, None, rin
    else:
        rin = rng.uniform(-1.5, 1.5, (E, IC)).astype(np.float32)
        re_np = rng.integers(0, E, m).astype(np.int32)
        re, rin_rows = torch.from_numpy(re_np).to(DEV), rin[re_np]
    got = ops().scaled_had(x, torch.from_numpy(rin).to(DEV), re)
    want = R.input_transform(v, rin_rows)
    assert np.array_equal(bits16(got), want.view(np.uint16))
    if dtype == torch.float32:
        # the same rows rounded to f16 first give a different transform
        pre = R.input_transform(v.astype(np.float16), rin_rows)
        assert not np.array_equal(pre.view(np.uint16), want.view(np.uint16))


def _linear_case(rng, ic, oc, K):
    code = rng.integers(-32768, 32768, size=(ic // 16, oc // 16, 16 * K), dtype=np.int16)
    rin = rng.choice([-1.0, 1.0], ic).astype(np.float16)
    rout = (rng.choice([-1.0, 1.0], oc) * rng.uniform(0.5, 1.5, oc) * 1e-2).astype(np.float16)
    bias = (rng.standard_normal(oc) * 0.05).astype(np.float16)
    return code, rin, rout, bias


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("m", [1, 4, 11, 24])
def test_linear_module_typed_rows(dtype, m, monkeypatch):
    """EschaLinear on bf16 / f32 rows: output in the input's dtype; the
    order-exact module bit-exact against the oracle's dense_linear on the same
    float32 rows (ordered sum), the default module within 2e-3 of each row's
    max against the float64 product."""
    from escha_mlx_amd.dense import EschaLinear, EschaWeight
    rng = np.random.default_rng(100 + m)
    ic, oc, K = 1024, 768, 2
    code, rin, rout, bias = _linear_case(rng, ic, oc, K)
    w = EschaWeight(code, rin, rout, device=DEV)
    v, x = _rows(rng, (m, ic), dtype)
    rin32, rout32 = rin.astype(np.float32), rout.astype(np.float32)
    monkeypatch.setenv("ESCHA_HIP_EXACT", "1")
    monkeypatch.setenv("ESCHA_MLX_DENSE_MAT", "0")  # 16+ rows: the order-exact rows kernel
    y_exact = EschaLinear(w, bias=bias)(x)
    assert y_exact.dtype == dtype
    want = R.dense_linear(v, code, rin32, rout32, K, bias=bias, ordered=True)
    assert np.array_equal(y_exact.float().cpu().numpy(),
                          torch.from_numpy(want.astype(np.float32)).to(dtype).float().numpy())
    monkeypatch.setenv("ESCHA_HIP_EXACT", "0")
    monkeypatch.delenv("ESCHA_MLX_DENSE_MAT")
    y = EschaLinear(w, bias=bias)(x)
    assert y.dtype == dtype
    wb = R.reconstruct(code, ic, oc, K)
    xh = R.input_transform(v, rin32)
    exact = R.h128(R.gemv_f64(xh, wb).astype(np.float32)) * R.RS * rout32 + bias.astype(np.float32)
    got = y.float().cpu().numpy()
    # the output is rounded to f16 (the contract) and then to bf16 for bf16 rows
    tol = 2e-3 if dtype == torch.float32 else 8e-3
    err = (np.abs(got - exact).max(axis=1) / np.abs(exact).max(axis=1)).max()
    assert err < tol, err
    if dtype == torch.float32:
        assert not torch.equal(EschaLinear(w, bias=bias)(x.half()).float(), y)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("exact", [False, True], ids=["fused", "exact"])
def test_moe_experts_typed_rows(dtype, exact, monkeypatch):
    """The routed expert path on bf16 / f32 token rows: the f16 routed sum
    against the oracle's routed block on the same float32 rows (1e-3 of the
    max through the order-exact chain, whose SwiGLU uses the device expf;
    5e-3 otherwise).  f32 rows give another result than the same rows
    rounded to f16 first."""
    E, H, I, K_gu, K_dn, T, k = 32, 512, 256, 2, 3, 3, 4
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 321)
    rng = np.random.default_rng(322)
    v, x = _rows(rng, (T, H), dtype)
    c = dict(c, x=v)
    blk = _block(c, E, k, K_gu, K_dn, monkeypatch, exact)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    y = blk(x, ids, sc)
    assert y.dtype == torch.float16
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np))
    got = y.cpu().numpy()
    if exact:
        # the chain's SwiGLU uses the device expf: one f16 ulp of h may move
        assert np.abs(got.astype(np.float32) - want.astype(np.float32)).max() / \
            np.abs(want.astype(np.float32)).max() < 1e-3
    else:
        assert np.abs(got.astype(np.float32) - want.astype(np.float32)).max() / \
            np.abs(want.astype(np.float32)).max() < 5e-3
    if dtype == torch.float32:
        assert not torch.equal(blk(x.half(), ids, sc), y)
