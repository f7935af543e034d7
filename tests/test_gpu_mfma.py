"""GPU parity of the matrix-core coded GEMM (esc_gemm_mfma, A14).

The kernel reassociates the float32 sum, so it is held to the two properties
the reference holds its matrix GEMM to (tests/test_dense_linear.py:486-524 of
escha-mlx): close to the order-exact row kernel (max |diff| / mean |ref| <
1e-3) and bit-identical run to run.  One-hot inputs leave one non-zero term
per output, so there the result must equal the decoded weight bit-for-bit,
which pins the decode, the operand layouts and the store map exactly.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not has_gpu(), reason="needs a ROCm GPU")]

DEV = "cuda"
MAT_TOL = 1e-3


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def ops():
    from escha_mlx_amd import ops as o
    return o


def _code(rng, ic, oc, K):
    u32 = rng.integers(0, 2**32, size=(ic // 16, oc // 16, 8 * K), dtype=np.uint64).astype(np.uint32)
    return u32, torch.from_numpy(u32.view(np.int32)).to(DEV)


def _dev_ratio(ref: torch.Tensor, got: torch.Tensor) -> float:
    return float((ref - got).abs().max()) / float(ref.abs().mean())


# the reference's own shapes and row counts (16 = one R=16 group, 17/33 = tails),
# plus a two-row-block case with an XCD-mapped column count (OC/128 = 8)
@pytest.mark.parametrize("ic,oc,K,m", [(256, 384, 2, 16), (256, 384, 2, 17), (256, 384, 2, 33),
                                       (512, 640, 3, 16), (512, 640, 3, 17), (512, 640, 3, 33),
                                       (1024, 1024, 2, 300), (1024, 1024, 3, 300),
                                       # OC a multiple of 256 (the direct-A kernel) at shapes for
                                       # which a 256-CU device picks 2, 4, 6 and 8 row blocks
                                       (512, 2048, 3, 50), (256, 4096, 2, 600), (256, 4096, 2, 1025),
                                       (256, 8192, 3, 900)])
def test_gemm_mat_close_to_rows_and_deterministic(ic, oc, K, m):
    rng = np.random.default_rng(909 + m + K)
    _, code = _code(rng, ic, oc, K)
    xh = torch.from_numpy((rng.standard_normal((m, ic)) * 0.3).astype(np.float16)).to(DEV)
    ref = ops().dense_gemm_rows(xh, code, K, ic, oc, 16)
    got = ops().dense_gemm_mat(xh, code, K, ic, oc)
    dev = _dev_ratio(ref, got)
    print(f"K={K} m={m} {ic}x{oc}: max|diff|/mean|ref| = {dev:.2e}")
    assert dev < MAT_TOL, f"K={K} m={m} deviates {dev:.2e}"
    again = ops().dense_gemm_mat(xh, code, K, ic, oc)
    assert torch.equal(got.view(torch.int32), again.view(torch.int32)), "not reproducible"


@pytest.mark.parametrize("K,ic,oc,m", [(2, 512, 1024, 300), (3, 512, 640, 70), (2, 2048, 128, 257),
                                       (3, 1024, 2048, 75), (2, 256, 4096, 600), (3, 256, 8192, 900)])
def test_gemm_mat_one_hot_rows_are_decoded_weights(K, ic, oc, m):
    rng = np.random.default_rng(31 * K + m)
    u32, code = _code(rng, ic, oc, K)
    k_of_row = rng.integers(0, ic, size=m)
    x = np.zeros((m, ic), np.float16)
    x[np.arange(m), k_of_row] = 1.0
    got = ops().dense_gemm_mat(torch.from_numpy(x).to(DEV), code, K, ic, oc).cpu().numpy()
    w = R.reconstruct(u32, ic, oc, K)
    assert np.array_equal(got, w[k_of_row].astype(np.float32))


@pytest.mark.parametrize("K,ic,oc,m", [(2, 2048, 1024, 260), (3, 1024, 2048, 64)])
def test_gemm_mat_vs_oracle_f64(K, ic, oc, m):
    rng = np.random.default_rng(5 + K)
    u32, code = _code(rng, ic, oc, K)
    xh = (rng.standard_normal((m, ic)) * 0.3).astype(np.float16)
    got = ops().dense_gemm_mat(torch.from_numpy(xh).to(DEV), code, K, ic, oc).cpu().numpy()
    ref = xh.astype(np.float64) @ R.reconstruct(u32, ic, oc, K).astype(np.float64)
    dev = np.abs(ref - got).max() / np.abs(ref).mean()
    print(f"K={K} {ic}x{oc} m={m}: max|diff|/mean|f64| = {dev:.2e}")
    assert dev < MAT_TOL


def test_dense_module_prefill_uses_matrix_path(monkeypatch):
    """EschaLinear at >= 16 rows: matrix path by default, within tolerance of
    the order-exact path (ESCHA_MLX_DENSE_MAT=0) after the output transform."""
    from escha_mlx_amd.dense import EschaLinear, EschaWeight
    rng = np.random.default_rng(77)
    ic, oc, K = 512, 1024, 3
    code = rng.integers(-32768, 32768, size=(ic // 16, oc // 16, 16 * K), dtype=np.int16)
    rin = np.where(rng.random(ic) < 0.5, -1.0, 1.0).astype(np.float16)
    rout = (np.where(rng.random(oc) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, oc) * 1e-2).astype(np.float16)
    x = torch.from_numpy(rng.standard_normal((48, ic)).astype(np.float16)).to(DEV)
    w = EschaWeight(code, rin, rout, device=DEV)
    monkeypatch.delenv("ESCHA_MLX_DENSE_MAT", raising=False)
    y_mat = EschaLinear(w)(x)
    monkeypatch.setenv("ESCHA_MLX_DENSE_MAT", "0")
    y_rows = EschaLinear(w)(x)
    d = (y_mat.float() - y_rows.float()).abs().max() / y_rows.float().abs().mean()
    assert float(d) < 5e-3


# ---- esc_gemm_mfma_out: the many-row GEMM with its output transform (one
# launch for OC a multiple of 256, else GEMM into the workspace + transform)
OUT_SHAPES = [(2, 512, 5120, 2048), (3, 1024, 3072, 2100), (3, 512, 640, 70), (2, 256, 384, 33),
              (2, 1024, 1024, 300)]


def _rout(rng, oc):
    return (rng.choice([-1.0, 1.0], oc) * rng.uniform(0.5, 1.5, oc) * 1e-2).astype(
        np.float16).astype(np.float32)


@pytest.mark.parametrize("K,ic,oc,m", OUT_SHAPES)
def test_gemm_out_one_hot_rows_exact(K, ic, oc, m):
    """One non-zero input per row: each output row is the oracle's output
    transform of v * W[k] bit-for-bit, with and without bias."""
    rng = np.random.default_rng(41 * K + m)
    u32, code = _code(rng, ic, oc, K)
    rout = _rout(rng, oc)
    bias = (rng.standard_normal(oc) * 0.05).astype(np.float16)
    k_of_row = rng.integers(0, ic, size=m)
    v = rng.choice([-1.5, 0.75, 1.0, 2.0], size=m).astype(np.float16)
    xh = np.zeros((m, ic), np.float16)
    xh[np.arange(m), k_of_row] = v
    w = R.reconstruct(u32, ic, oc, K)
    mid = v.astype(np.float32)[:, None] * w[k_of_row].astype(np.float32)
    want = R.output_transform(mid, rout)
    xh_d, rout_d = torch.from_numpy(xh).to(DEV), torch.from_numpy(rout).to(DEV)
    y = ops().gemm_mfma_out(xh_d, code, rout_d, K, ic, oc).cpu().numpy()
    assert np.array_equal(y.view(np.uint16), want.view(np.uint16))
    yb = ops().gemm_mfma_out(xh_d, code, rout_d, K, ic, oc,
                             bias=torch.from_numpy(bias).to(DEV)).cpu().numpy()
    wantb = (want.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    assert np.array_equal(yb.view(np.uint16), wantb.view(np.uint16))


@pytest.mark.parametrize("K,ic,oc,m", OUT_SHAPES[:4])
def test_gemm_out_vs_f64_and_two_launches(K, ic, oc, m):
    """Random rows: within the float16 tolerance of the float64 product after
    the output transform, and bit-identical to esc_gemm_mfma followed by
    esc_output_transform (the same float32 order)."""
    rng = np.random.default_rng(17 * K + m)
    u32, code = _code(rng, ic, oc, K)
    rout = _rout(rng, oc)
    xh = (rng.standard_normal((m, ic)) * 0.3).astype(np.float16)
    xh_d, rout_d = torch.from_numpy(xh).to(DEV), torch.from_numpy(rout).to(DEV)
    y = ops().gemm_mfma_out(xh_d, code, rout_d, K, ic, oc)
    exact = R.h128(xh.astype(np.float64) @ R.reconstruct(u32, ic, oc, K).astype(np.float64)) \
        * R.RS * rout
    got = y.cpu().numpy().astype(np.float64)
    err = (np.abs(got - exact).max(axis=1) / np.abs(exact).max(axis=1)).max()
    assert err < 2e-3, err
    two = ops().scaled_had_out(ops().dense_gemm_mat(xh_d, code, K, ic, oc), rout_d, None)
    assert torch.equal(y, two)


def test_linear_many_rows_is_transform_then_gemm_out():
    """esc_linear from 16 rows = esc_input_transform then esc_gemm_mfma_out,
    bit-identical."""
    rng = np.random.default_rng(23)
    K, ic, oc, m = 2, 512, 5120, 2048
    u32, code = _code(rng, ic, oc, K)
    rin = rng.choice([-1.0, 1.0], ic).astype(np.float16).astype(np.float32)
    rout = _rout(rng, oc)
    bias = torch.from_numpy((rng.standard_normal(oc) * 0.05).astype(np.float16)).to(DEV)
    x = torch.from_numpy(rng.standard_normal((m, ic)).astype(np.float16)).to(DEV)
    rin_d, rout_d = torch.from_numpy(rin).to(DEV), torch.from_numpy(rout).to(DEV)
    y = ops().linear(x, code, rin_d, rout_d, K, ic, oc, bias=bias)
    want = ops().gemm_mfma_out(ops().scaled_had(x, rin_d, None), code, rout_d, K, ic, oc, bias=bias)
    assert torch.equal(y, want)
