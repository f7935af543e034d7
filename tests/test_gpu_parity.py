"""GPU parity: HIP kernels through the C ABI vs the NumPy oracle.

Bar: bit-exact for decode, transforms, routing ids, grouping and every
order-exact GEMV / GEMM (the reference kernels' float32 order); the split-K
GEMV and the fused MoE path are held to a float16 tolerance against float64
(and to bit-exactness where the sum has one non-zero term: one-hot inputs).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_np as R

from .conftest import has_gpu, sha256

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


def bits16(t):
    return t.cpu().numpy().view(np.uint16)


def rand_code(rng, shape_words):
    return rng.integers(0, 2**32, size=shape_words, dtype=np.uint64).astype(np.uint32)


def dcode(u32: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(u32).view(np.int32)).to(DEV)


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("which", ["k2", "k3"])
def test_decode_tiles_bit_exact_vs_goldens(which, lut, k2_golden, k3_golden):
    packed, meta, head = k2_golden if which == "k2" else k3_golden
    K = 2 if which == "k2" else 3
    ic, oc = meta["shape"]
    w = ops().decode_tiles(ops().to_device_code(packed, DEV), K, ic, oc, lut=lut)
    got = w.cpu().numpy()
    assert np.array_equal(got[: meta["head_rows"]].view(np.uint16), head.view(np.uint16))
    assert sha256(got) == meta["sha256"], "decoded golden differs"


@pytest.mark.parametrize("K", [2, 3])
def test_decode_hash_equals_lut_equals_oracle_random(K):
    rng = np.random.default_rng(42 + K)
    code = rand_code(rng, (16, 24, 8 * K))
    d = dcode(code)
    a = bits16(ops().decode_tiles(d, K, 256, 384, lut=False))
    b = bits16(ops().decode_tiles(d, K, 256, 384, lut=True))
    want = R.reconstruct(code, 256, 384, K).view(np.uint16)
    assert np.array_equal(a, want) and np.array_equal(b, want)


# ---------------------------------------------------------------- transforms

@pytest.mark.parametrize("m,IC,E", [(8, 512, 256), (96, 2048, 64), (3, 128, 1)])
def test_input_transform_bit_exact(m, IC, E):
    rng = np.random.default_rng(m * 7 + IC)
    rows = rng.standard_normal((m, IC)).astype(np.float16)
    rin = rng.standard_normal((E, IC)).astype(np.float32)
    re = rng.integers(0, E, size=m).astype(np.int32)
    got = ops().scaled_had(torch.from_numpy(rows).to(DEV), torch.from_numpy(rin).to(DEV),
                           torch.from_numpy(re).to(DEV))
    want = R.input_transform(rows, rin[re])
    assert np.array_equal(bits16(got), want.view(np.uint16))
    # dense variant
    got_d = ops().scaled_had(torch.from_numpy(rows).to(DEV), torch.from_numpy(rin[0]).to(DEV), None)
    assert np.array_equal(bits16(got_d), R.input_transform(rows, rin[0]).view(np.uint16))


@pytest.mark.parametrize("m,OC,E", [(8, 1024, 256), (33, 384, 7)])
def test_output_transform_bit_exact(m, OC, E):
    rng = np.random.default_rng(m + OC)
    mid = (rng.standard_normal((m, OC)) * 5).astype(np.float32)
    rout = (rng.standard_normal((E, OC)) * 0.01).astype(np.float32)
    re = rng.integers(0, E, size=m).astype(np.int32)
    got = ops().scaled_had_out(torch.from_numpy(mid).to(DEV), torch.from_numpy(rout).to(DEV),
                               torch.from_numpy(re).to(DEV))
    assert np.array_equal(bits16(got), R.output_transform(mid, rout[re]).view(np.uint16))


def test_transforms_match_reference_vectors(ref_vectors):
    v = ref_vectors
    got = ops().scaled_had(torch.from_numpy(v["in_x"]).to(DEV), torch.from_numpy(v["in_rin"]).to(DEV), None)
    assert np.array_equal(bits16(got), v["in_y"].view(np.uint16))
    got = ops().scaled_had_out(torch.from_numpy(v["out_mid"]).to(DEV),
                               torch.from_numpy(v["out_rout"]).to(DEV), None)
    assert np.array_equal(bits16(got), v["out_y"].view(np.uint16))


def test_swiglu_vs_reference_vectors(ref_vectors):
    x = ref_vectors["swiglu_x"]
    got = bits16(ops().swiglu(torch.from_numpy(x).to(DEV)))
    want = ref_vectors["swiglu_y"].view(np.uint16)
    # device expf vs numpy exp: identical f16 except where an f32 ulp crosses a tie
    mism = int((got != want).sum())
    assert mism <= max(1, got.size // 1000), mism
    g = got.view(np.float16).astype(np.float32)
    w = want.view(np.float16).astype(np.float32)
    assert np.abs(g - w).max() <= np.abs(w).max() * 2 ** -10


# ---------------------------------------------------------------- order-exact GEMV

def _expert_stack(rng, K, ic, oc, E):
    return rand_code(rng, (E, ic // 16, oc // 16, 8 * K))


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,IC,OC", [(2, 2048, 1024), (3, 512, 2048)])
def test_moe_gemv_bit_exact_mixed_experts(K, IC, OC, lut):
    """Expert-stride indexing with 0 and E-1 included (reference tests/test_metal.py:46-72),
    held to bit-exactness against the oracle's kernel-order GEMV."""
    rng = np.random.default_rng(K)
    E = 4
    codes = _expert_stack(rng, K, IC, OC, E)
    xh = (rng.standard_normal((8, IC)) * 0.05).astype(np.float16)
    re = np.array([0, E - 1, 1, 2, E - 1, 0, 2, 1], dtype=np.int32)
    mid = ops().moe_gemv(torch.from_numpy(xh).to(DEV), dcode(codes), torch.from_numpy(re).to(DEV),
                         K, IC, OC, lut=lut).cpu().numpy()
    w = [R.reconstruct(codes[e], IC, OC, K) for e in range(E)]
    for r in range(8):
        want = R.gemv_ordered(xh[r:r + 1], w[re[r]])[0]
        assert np.array_equal(mid[r].view(np.uint32), want.view(np.uint32)), r


def test_dense_gemv_golden_stream_bit_exact(k2_golden):
    packed, meta, _ = k2_golden
    ic, oc = meta["shape"]
    rng = np.random.default_rng(0)
    xh = rng.standard_normal((3, ic)).astype(np.float16)
    mid = ops().dense_gemv(torch.from_numpy(xh).to(DEV), ops().to_device_code(packed, DEV), 2, ic, oc)
    want = R.gemv_ordered(xh, R.reconstruct(packed, ic, oc, 2))
    assert np.array_equal(mid.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("R_", [2, 3, 4, 12])
def test_gemm_rows_bit_identical_to_per_row(R_):
    """Row blocking changes only the loop nest (reference tests/test_blocked.py:69-161)."""
    from escha_mlx_amd import moe
    rng = np.random.default_rng(R_)
    K, IC, OC, E, m = 2, 512, 256, 16, 45
    codes = _expert_stack(rng, K, IC, OC, E)
    re = rng.integers(0, E, size=m).astype(np.int32)
    re[:9] = 3  # skew: one expert with many rows
    xh = rng.standard_normal((m, IC)).astype(np.float16)
    d_xh, d_code, d_re = torch.from_numpy(xh).to(DEV), dcode(codes), torch.from_numpy(re).to(DEV)
    per_row = ops().moe_gemv(d_xh, d_code, d_re, K, IC, OC).cpu().numpy()
    ng = moe.n_groups_bound(m, E, R_)
    rows_idx, group_expert = moe.build_groups(d_re, E, R_, ng)
    ri, ge = R.build_groups(re, E, R_, ng)
    assert np.array_equal(rows_idx.cpu().numpy(), ri) and np.array_equal(group_expert.cpu().numpy(), ge)
    xh_pad = torch.cat([d_xh, torch.zeros((1, IC), dtype=torch.float16, device=DEV)])
    mid = ops().moe_gemm_rows(xh_pad, d_code, rows_idx, group_expert, K, IC, OC, R_, m).cpu().numpy()
    assert np.array_equal(mid[:m].view(np.uint32), per_row.view(np.uint32))
    # and directly against the oracle's kernel-order GEMV, row by row
    w = {e: R.reconstruct(codes[e], IC, OC, K) for e in np.unique(re)}
    for r in range(m):
        want = R.gemv_ordered(xh[r:r + 1], w[re[r]])[0]
        assert np.array_equal(mid[r].view(np.uint32), want.view(np.uint32)), r


@pytest.mark.parametrize("m", [1, 63, 64, 65, 256, 1000, 1025, 2500])
@pytest.mark.parametrize("E,R_", [(8, 2), (256, 8), (256, 3)])
def test_build_groups_matches_oracle(m, E, R_):
    """Stable expert grouping across waves and 1024-row chunks (rows of one
    expert keep their order) against the oracle's brute-force model."""
    from escha_mlx_amd import moe
    rng = np.random.default_rng(m * 7 + E + R_)
    re = rng.integers(0, E, size=m).astype(np.int32)
    re[: m // 3] = E - 1  # skew: one expert owns a third of the rows
    ng = moe.n_groups_bound(m, E, R_)
    rows_idx, group_expert = moe.build_groups(torch.from_numpy(re).to(DEV), E, R_, ng)
    ri, ge = R.build_groups(re, E, R_, ng)
    assert np.array_equal(rows_idx.cpu().numpy(), ri)
    assert np.array_equal(group_expert.cpu().numpy(), ge)


@pytest.mark.parametrize("R_", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("m", [1, 5, 17])
def test_dense_rows_bit_identical_to_gemv(R_, m):
    rng = np.random.default_rng(R_ * 100 + m)
    K, IC, OC = 3, 256, 384
    code = rand_code(rng, (IC // 16, OC // 16, 8 * K))
    xh = rng.standard_normal((m, IC)).astype(np.float16)
    d_xh, d_code = torch.from_numpy(xh).to(DEV), dcode(code)
    a = ops().dense_gemv(d_xh, d_code, K, IC, OC).cpu().numpy()
    b = ops().dense_gemm_rows(d_xh, d_code, K, IC, OC, R_).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), R.gemv_ordered(xh, R.reconstruct(code, IC, OC, K)).view(np.uint32))


@pytest.mark.parametrize("R_", [1, 2, 4, 8])
def test_dense_rows_out_bit_identical_to_chain(R_):
    rng = np.random.default_rng(9 + R_)
    K, IC, OC, m = 2, 384, 256, 7
    code = rand_code(rng, (IC // 16, OC // 16, 8 * K))
    xh = rng.standard_normal((m, IC)).astype(np.float16)
    rout = (rng.standard_normal(OC) * 0.01).astype(np.float32)
    d = ops().dense_gemm_rows_direct_out(torch.from_numpy(xh).to(DEV), dcode(code),
                                         torch.from_numpy(rout).to(DEV), K, IC, OC, R_)
    want = R.output_transform(R.gemv_ordered(xh, R.reconstruct(code, IC, OC, K)), rout)
    assert np.array_equal(bits16(d), want.view(np.uint16))


# ---------------------------------------------------------------- split-K GEMV

def _fast_case(K, IC, OC, E, m, seed):
    rng = np.random.default_rng(seed)
    codes = _expert_stack(rng, K, IC, OC, E)
    rout = (rng.choice([-1.0, 1.0], (E, OC)) * rng.uniform(0.5, 1.5, (E, OC)) * 1e-2).astype(np.float32)
    re = rng.integers(0, E, size=m).astype(np.int32)
    return rng, codes, rout, re


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,IC,OC", [(2, 2048, 1024), (2, 512, 2048), (3, 512, 2048), (3, 2048, 1024)])
def test_fast_gemv_one_hot_bit_exact(K, IC, OC, lut):
    """One non-zero input per row: every reassociated sum is exact, so the fused
    decode + output transform must equal the oracle bit-for-bit."""
    rng, codes, rout, re = _fast_case(K, IC, OC, 3, 5, 100 + K + IC)
    xh = np.zeros((5, IC), np.float16)
    hot = rng.integers(0, IC, size=5)
    for r in range(5):
        xh[r, hot[r]] = np.float16(rng.choice([1.0, -2.0, 0.5]))
    out = ops().gemv_fast_out(torch.from_numpy(xh).to(DEV), dcode(codes), torch.from_numpy(re).to(DEV),
                              torch.from_numpy(rout).to(DEV), K, IC, OC, lut=lut)
    w = [R.reconstruct(codes[e], IC, OC, K) for e in range(3)]
    for r in range(5):
        mid = xh[r, hot[r]].astype(np.float32) * w[re[r]][hot[r]].astype(np.float32)
        want = R.output_transform(mid[None], rout[re[r]])[0]
        assert np.array_equal(bits16(out)[r], want.view(np.uint16)), r


@pytest.mark.parametrize("K,IC,OC,m", [(2, 2048, 1024, 8), (2, 512, 2048, 8), (3, 5120, 1024, 1),
                                       (3, 1024, 2048, 4)])
def test_fast_gemv_tolerance_vs_f64(K, IC, OC, m):
    rng, codes, rout, re = _fast_case(K, IC, OC, 4, m, K * 31 + m)
    xh = rng.standard_normal((m, IC)).astype(np.float16)
    out = ops().gemv_fast_out(torch.from_numpy(xh).to(DEV), dcode(codes), torch.from_numpy(re).to(DEV),
                              torch.from_numpy(rout).to(DEV), K, IC, OC).cpu().numpy().astype(np.float32)
    worst = 0.0
    for r in range(m):
        w = R.reconstruct(codes[re[r]], IC, OC, K)
        mid64 = R.gemv_f64(xh[r:r + 1], w)[0]
        exact = (R.h128(mid64[None].astype(np.float32)) * R.RS * rout[re[r]])[0]
        err = np.abs(out[r] - exact).max() / np.abs(exact).max()
        worst = max(worst, err)
    # f16 output rounding (2^-11 relative) + f32 reassociation: 2e-3 of the row max
    assert worst < 2e-3, worst


def test_fast_gemv_deterministic():
    rng, codes, rout, re = _fast_case(2, 2048, 1024, 8, 8, 5)
    xh = torch.from_numpy(rng.standard_normal((8, 2048)).astype(np.float16)).to(DEV)
    args = (xh, dcode(codes), torch.from_numpy(re).to(DEV), torch.from_numpy(rout).to(DEV), 2, 2048, 1024)
    first = bits16(ops().gemv_fast_out(*args))
    for _ in range(8):
        assert np.array_equal(bits16(ops().gemv_fast_out(*args)), first)


@pytest.mark.parametrize("lut", [False, True], ids=["hash", "lut"])
@pytest.mark.parametrize("K,IC,OC,m,R_", [(2, 2048, 1024, 5, 4), (3, 512, 2048, 8, 8),
                                          (2, 1024, 384, 3, 2), (3, 1024, 640, 13, 8)])
def test_fast_rows_one_hot_bit_exact(K, IC, OC, m, R_, lut):
    """R rows per decode: one non-zero input per row keeps every sum exact."""
    rng = np.random.default_rng(7 * K + m + R_)
    code = _expert_stack(rng, K, IC, OC, 1)[0]
    rout = (rng.choice([-1.0, 1.0], OC) * rng.uniform(0.5, 1.5, OC) * 1e-2).astype(np.float32)
    xh = np.zeros((m, IC), np.float16)
    hot = rng.integers(0, IC, size=m)
    for r in range(m):
        xh[r, hot[r]] = np.float16(rng.choice([1.0, -2.0, 0.5]))
    out = ops().dense_gemm_rows_fast_out(torch.from_numpy(xh).to(DEV), dcode(code),
                                         torch.from_numpy(rout).to(DEV), K, IC, OC, R_, lut=lut)
    w = R.reconstruct(code, IC, OC, K)
    for r in range(m):
        mid = xh[r, hot[r]].astype(np.float32) * w[hot[r]].astype(np.float32)
        want = R.output_transform(mid[None], rout)[0]
        assert np.array_equal(bits16(out)[r], want.view(np.uint16)), r


@pytest.mark.parametrize("K,IC,OC,m,R_", [(2, 5120, 1024, 4, 4), (3, 1024, 2048, 7, 8),
                                          (3, 2048, 512, 2, 2)])
def test_fast_rows_tolerance_vs_f64_and_deterministic(K, IC, OC, m, R_):
    rng = np.random.default_rng(K * 17 + m)
    code = _expert_stack(rng, K, IC, OC, 1)[0]
    rout = (rng.choice([-1.0, 1.0], OC) * rng.uniform(0.5, 1.5, OC) * 1e-2).astype(np.float32)
    xh = rng.standard_normal((m, IC)).astype(np.float16)
    args = (torch.from_numpy(xh).to(DEV), dcode(code), torch.from_numpy(rout).to(DEV), K, IC, OC, R_)
    out = ops().dense_gemm_rows_fast_out(*args)
    w = R.reconstruct(code, IC, OC, K)
    exact = R.h128(R.gemv_f64(xh, w).astype(np.float32)) * R.RS * rout
    got = out.cpu().numpy().astype(np.float32)
    err = (np.abs(got - exact).max(axis=1) / np.abs(exact).max(axis=1)).max()
    assert err < 2e-3, err
    assert np.array_equal(bits16(ops().dense_gemm_rows_fast_out(*args)), bits16(out))


# ---------------------------------------------------------------- routing / MoE

def test_route_topk_matches_oracle(ref_vectors):
    lg = ref_vectors["route_logits"]
    ids, sc = ops().route_topk(torch.from_numpy(lg).to(DEV), 8)
    assert np.array_equal(ids.cpu().numpy(), ref_vectors["route_ids"])
    assert np.allclose(sc.cpu().numpy(), ref_vectors["route_scores"], rtol=2e-6, atol=0)
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((32, 256)).astype(np.float32)
    lg[5, :] = 0.25  # all tied: lowest ids win
    ids, sc = ops().route_topk(torch.from_numpy(lg).to(DEV), 8)
    want_ids, want_sc = R.route_topk(lg, 8)
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.allclose(sc.cpu().numpy(), want_sc, rtol=2e-6, atol=0)


def _moe_case(E, H, I, K_gu, K_dn, T, k, seed):
    rng = np.random.default_rng(seed)
    gu_code = rand_code(rng, (E, H // 16, 2 * I // 16, 8 * K_gu))
    dn_code = rand_code(rng, (E, I // 16, H // 16, 8 * K_dn))
    gu_rin = rng.choice([-1.0, 1.0], (E, H)).astype(np.float32)
    dn_rin = rng.choice([-1.0, 1.0], (E, I)).astype(np.float32)
    gu_rout = (rng.choice([-1.0, 1.0], (E, 2 * I)) * rng.uniform(0.5, 1.5, (E, 2 * I)) * 4e-2).astype(np.float32)
    dn_rout = (rng.choice([-1.0, 1.0], (E, H)) * rng.uniform(0.5, 1.5, (E, H)) * 4e-2).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    return dict(gu_code=gu_code, dn_code=dn_code, gu_rin=gu_rin, dn_rin=dn_rin, gu_rout=gu_rout,
                dn_rout=dn_rout, x=x, logits=logits)


def _block(c, E, k, K_gu, K_dn, monkeypatch, exact):
    from escha_mlx_amd import moe
    monkeypatch.setenv("ESCHA_HIP_EXACT", "1" if exact else "0")
    gu = moe.EschaExperts.from_device(dcode(c["gu_code"]), torch.from_numpy(c["gu_rin"]).to(DEV),
                                      torch.from_numpy(c["gu_rout"]).to(DEV), K_gu)
    dn = moe.EschaExperts.from_device(dcode(c["dn_code"]), torch.from_numpy(c["dn_rin"]).to(DEV),
                                      torch.from_numpy(c["dn_rout"]).to(DEV), K_dn)
    return moe.EschaMoEExperts(gu, dn, E, k)


def _oracle_moe(c, ids, sc, E, H, I, K_gu, K_dn, used):
    w_gu = np.zeros((E, H, 2 * I), np.float16)
    w_dn = np.zeros((E, I, H), np.float16)
    for e in used:
        w_gu[e] = R.reconstruct(c["gu_code"][e], H, 2 * I, K_gu)
        w_dn[e] = R.reconstruct(c["dn_code"][e], I, H, K_dn)
    return R.moe_routed(c["x"], ids, sc, {"w": w_gu, "rin": c["gu_rin"], "rout": c["gu_rout"]},
                        {"w": w_dn, "rin": c["dn_rin"], "rout": c["dn_rout"]}, K_gu, K_dn,
                        ordered=True)


@pytest.mark.parametrize("exact", [False, True], ids=["fused", "exact"])
@pytest.mark.parametrize("E,H,I,K_gu,K_dn,T,k", [(16, 256, 128, 2, 2, 1, 8), (32, 512, 256, 2, 3, 3, 4)])
def test_moe_expert_path_vs_oracle(E, H, I, K_gu, K_dn, T, k, exact, monkeypatch):
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, E + H + T)
    blk = _block(c, E, k, K_gu, K_dn, monkeypatch, exact)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    y = blk(torch.from_numpy(c["x"]).to(DEV), ids, sc).cpu().numpy()
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np))
    g, w = y.astype(np.float32), want.astype(np.float32)
    rel = np.abs(g - w).max() / np.abs(w).max()
    # exact chain: same order and rounding points; swiglu's exp may differ by an
    # f32 ulp (device expf vs numpy exp), which one flipped h element spreads
    # over the down leg's outputs — bit-exactness is pinned stage-wise below.
    assert rel < (1e-3 if exact else 5e-3), rel


@pytest.mark.parametrize("K_gu,K_dn", [(2, 2), (2, 3)])
def test_moe_exact_chain_stagewise_bit_exact(K_gu, K_dn):
    """Every stage of the reference chain bit-exact vs the oracle; swiglu within
    one f16 ulp; the down leg and the combine are then fed the device's h."""
    E, H, I, T, k = 32, 512, 256, 3, 4
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 91 + K_dn)
    o = ops()
    ids, sc = o.route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    re_np = ids_np.reshape(-1).astype(np.int32)
    re = torch.from_numpy(re_np).to(DEV)
    rows = np.repeat(c["x"], k, axis=0)
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    xh = o.scaled_had(dv(rows), dv(c["gu_rin"]), re)
    xh_ref = R.input_transform(rows, c["gu_rin"][re_np])
    assert np.array_equal(bits16(xh), xh_ref.view(np.uint16))
    mid = o.moe_gemv(xh, dcode(c["gu_code"]), re, K_gu, H, 2 * I).cpu().numpy()
    w_gu = {e: R.reconstruct(c["gu_code"][e], H, 2 * I, K_gu) for e in np.unique(re_np)}
    w_dn = {e: R.reconstruct(c["dn_code"][e], I, H, K_dn) for e in np.unique(re_np)}
    mid_ref = np.stack([R.gemv_ordered(xh_ref[r:r + 1], w_gu[re_np[r]])[0] for r in range(len(re_np))])
    assert np.array_equal(mid.view(np.uint32), mid_ref.view(np.uint32))
    gu16 = o.scaled_had_out(dv(mid), dv(c["gu_rout"]), re)
    gu16_ref = R.output_transform(mid_ref, c["gu_rout"][re_np])
    assert np.array_equal(bits16(gu16), gu16_ref.view(np.uint16))
    h = o.swiglu(gu16)
    h_np = h.cpu().numpy()
    ulps = np.abs(h_np.view(np.uint16).astype(np.int32) - R.swiglu(gu16_ref).view(np.uint16).astype(np.int32))
    assert ulps.max() <= 1
    xh2 = o.scaled_had(h, dv(c["dn_rin"]), re)
    xh2_ref = R.input_transform(h_np, c["dn_rin"][re_np])
    assert np.array_equal(bits16(xh2), xh2_ref.view(np.uint16))
    mid2 = o.moe_gemv(xh2, dcode(c["dn_code"]), re, K_dn, I, H).cpu().numpy()
    mid2_ref = np.stack([R.gemv_ordered(xh2_ref[r:r + 1], w_dn[re_np[r]])[0] for r in range(len(re_np))])
    assert np.array_equal(mid2.view(np.uint32), mid2_ref.view(np.uint32))
    d16 = o.scaled_had_out(dv(mid2), dv(c["dn_rout"]), re)
    d16_ref = R.output_transform(mid2_ref, c["dn_rout"][re_np])
    assert np.array_equal(bits16(d16), d16_ref.view(np.uint16))
    y = o.moe_combine(d16, sc.reshape(-1).contiguous(), k)
    w16 = sc_np.reshape(-1).astype(np.float16).astype(np.float32)
    contrib = d16_ref.astype(np.float32) * w16[:, None]
    y_ref = np.zeros((T, H), np.float32)
    for s in range(k):
        y_ref = y_ref + contrib[s::k]
    assert np.array_equal(bits16(y), y_ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("E,T,K_gu,K_dn,H", [(64, 9, 2, 3, 256), (16, 12, 3, 2, 256),
                                             (256, 9, 2, 2, 256), (16, 12, 2, 2, 384)],
                         ids=["grouped", "grouped_experts_over_8_rows", "per_row",
                              "grouped_partial_tile_group"])
def test_moe_multi_launch_path_vs_oracle(E, T, K_gu, K_dn, H, monkeypatch):
    """More rows than the one-launch path takes (T*k > 64): split-K chain, with
    rows of one expert sharing each decoded weight once rows >= experts
    (groups in the moe.build_groups layout), per row otherwise; deterministic,
    and repeat calls on one workspace agree."""
    I, k = 128, 8
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 5 + E)
    blk = _block(c, E, k, K_gu, K_dn, monkeypatch, exact=False)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    y = blk(x, ids, sc)
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
    got = y.cpu().numpy().astype(np.float32)
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
    assert torch.equal(blk(x, ids, sc), y)


@pytest.mark.parametrize("E,T,K_gu,K_dn,H,I", [(64, 9, 2, 2, 256, 128), (64, 12, 3, 2, 512, 256),
                                                 (32, 16, 2, 3, 384, 128), (256, 32, 2, 2, 2048, 512)],
                         ids=["k2", "gate_up_k3", "down_k3", "config4_shape"])
def test_moe_grouped_table_path_bit_identical_to_hash(E, T, K_gu, K_dn, H, I, monkeypatch):
    """The grouped chain with the table asked for runs the persistent
    k_gemv_rows_table (one workgroup per CU, the table staged once, waves over
    contiguous wave-item ranges): its partials are the hash kernel's bit for
    bit, so the whole path's output is; and both are within tolerance of the
    oracle.  Repeat calls on one workspace agree."""
    k = 8
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 40 + E + T)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    args = [dcode(c["gu_code"]), torch.from_numpy(c["gu_rin"]).to(DEV),
            torch.from_numpy(c["gu_rout"]).to(DEV), K_gu, dcode(c["dn_code"]),
            torch.from_numpy(c["dn_rin"]).to(DEV), torch.from_numpy(c["dn_rout"]).to(DEV), K_dn]
    ws = torch.zeros(ops().moe_expert_path_workspace(T, k, E, H, I), dtype=torch.uint8, device=DEV)
    y_hash = ops().moe_expert_path(x, ids, sc, *args, lut=False, ws=ws)
    y_tab = ops().moe_expert_path(x, ids, sc, *args, lut=True, ws=ws)
    assert torch.equal(y_tab, y_hash)
    assert torch.equal(ops().moe_expert_path(x, ids, sc, *args, lut=True, ws=ws), y_tab)
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
    got = y_tab.cpu().numpy().astype(np.float32)
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3


def test_moe_one_launch_status_and_reuse(monkeypatch):
    """The one persistent launch (k_moe_fused: H or I not a multiple of 512)
    never hits its bounded wait and leaves its counters zero: repeated calls on
    one workspace agree bit-for-bit and the status flag stays clear."""
    E, H, I, k = 64, 512, 256, 8
    c = _moe_case(E, H, I, 2, 2, 1, k, 12)
    blk = _block(c, E, k, 2, 2, monkeypatch, exact=False)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    first = bits16(blk(x, ids, sc))
    for _ in range(4):
        assert np.array_equal(bits16(blk(x, ids, sc)), first)
    ws = blk._ws[(1, x.device, False)]
    assert ops().moe_status(ws, 1, k, H, I) == 0


@pytest.mark.parametrize("E,H,I,K_gu,K_dn,T,k", [(256, 2048, 512, 2, 2, 1, 8),
                                                  (256, 2048, 512, 2, 2, 4, 8),
                                                  (64, 1024, 512, 2, 3, 8, 8)])
def test_moe_one_launch_entry_vs_oracle(E, H, I, K_gu, K_dn, T, k):
    """esc_moe_expert_path_one_launch at shapes the default runs as two
    launches (config 3's among them, and 64 routed rows, the most it takes):
    against the oracle, beside the two-launch default, bit-identical on repeat
    on one workspace (its counters left zero), and no bounded wait given up."""
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 5 * T + K_dn)
    o = ops()
    ids, sc = o.route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    args = (x, ids, sc, dcode(c["gu_code"]), torch.from_numpy(c["gu_rin"]).to(DEV),
            torch.from_numpy(c["gu_rout"]).to(DEV), K_gu, dcode(c["dn_code"]),
            torch.from_numpy(c["dn_rin"]).to(DEV), torch.from_numpy(c["dn_rout"]).to(DEV), K_dn)
    ws = torch.zeros(o.moe_expert_path_workspace(T, k, E, H, I), dtype=torch.uint8, device=DEV)
    one = o.moe_expert_path(*args, ws=ws, one_launch=True)
    first = bits16(one)
    for _ in range(3):
        assert np.array_equal(bits16(o.moe_expert_path(*args, ws=ws, one_launch=True)), first)
    assert o.moe_status(ws, T, k, H, I) == 0
    # the two-launch default on a workspace of its own (the plans differ)
    two = o.moe_expert_path(*args).cpu().numpy().astype(np.float32)
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
    scale = np.abs(want).max()
    got = one.cpu().numpy().astype(np.float32)
    assert np.isfinite(got).all()
    assert np.abs(got - want).max() / scale < 5e-3
    assert np.abs(two - want).max() / scale < 5e-3


def test_moe_one_launch_gave_up_wait_is_reported(monkeypatch):
    """Failure reporting of the one persistent launch, forced from the host:
    with a spin limit of 0 every down item's wait gives up at once (no wait
    runs, so the kernel still reaches its end), its outputs are NaN, and the
    next call on the device raises EschaWaitTimeout without running; the call
    after that matches the good output bit-for-bit, and the workspace's own
    flag still reads 1 once.  Read through esc_moe_status first instead, the
    failure is reported once and no call raises."""
    from escha_mlx_amd import _lib
    E, H, I, k = 64, 512, 256, 8
    c = _moe_case(E, H, I, 2, 2, 1, k, 13)
    blk = _block(c, E, k, 2, 2, monkeypatch, exact=False)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    good = bits16(blk(x, ids, sc))
    assert not np.isnan(good.view(np.float16)).any()
    ws = blk._ws[(1, x.device, False)]
    for via_status in (False, True):
        ops().set_moe_spin_limit(0)
        try:
            bad = blk(x, ids, sc).float().cpu()
        finally:
            ops().set_moe_spin_limit(-1)
        assert torch.isnan(bad).all()
        if via_status:
            assert ops().moe_status(ws, 1, k, H, I) == 1
        else:
            with pytest.raises(_lib.EschaWaitTimeout, match="bounded wait"):
                blk(x, ids, sc)
        assert np.array_equal(bits16(blk(x, ids, sc)), good)
        # the workspace's own flag keeps the failure until esc_moe_status reads it
        if not via_status:
            assert ops().moe_status(ws, 1, k, H, I) == 1
        assert ops().moe_status(ws, 1, k, H, I) == 0


def test_moe_module_one_launch_knob(monkeypatch):
    """ESCHA_HIP_MOE_ONE_LAUNCH=1: EschaMoEExperts takes the one-launch entry
    where it takes the shape (bit-identical to calling it directly) and the
    default elsewhere (above 64 routed rows)."""
    E, H, I, k = 64, 1024, 512, 8
    monkeypatch.setenv("ESCHA_HIP_MOE_ONE_LAUNCH", "1")
    for T in (2, 12):
        c = _moe_case(E, H, I, 2, 2, T, k, 31 + T)
        blk = _block(c, E, k, 2, 2, monkeypatch, exact=False)
        assert blk._one_launch
        ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
        x = torch.from_numpy(c["x"]).to(DEV)
        got = bits16(blk(x, ids, sc))
        one = T * k <= 64
        assert ops().moe_one_launch_takes(T, k, H, I) == one
        args = (x, ids, sc, dcode(c["gu_code"]), torch.from_numpy(c["gu_rin"]).to(DEV),
                torch.from_numpy(c["gu_rout"]).to(DEV), 2, dcode(c["dn_code"]),
                torch.from_numpy(c["dn_rin"]).to(DEV), torch.from_numpy(c["dn_rout"]).to(DEV), 2)
        want = bits16(ops().moe_expert_path(*args, one_launch=one))
        assert np.array_equal(got, want), T


def test_moe_one_launch_entry_gave_up_wait_is_reported():
    """The same failure reporting for esc_moe_expert_path_one_launch at a shape
    the default runs as two launches, forced from the host (spin limit 0: the
    kernel still reaches its end): NaN outputs, then either the next one-launch
    call raises EschaWaitTimeout without running or esc_moe_status reports the
    device-wide flag once; the call after that matches the good output."""
    from escha_mlx_amd import _lib
    E, H, I, k = 64, 1024, 512, 8
    c = _moe_case(E, H, I, 2, 2, 1, k, 17)
    o = ops()
    ids, sc = o.route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    args = (x, ids, sc, dcode(c["gu_code"]), torch.from_numpy(c["gu_rin"]).to(DEV),
            torch.from_numpy(c["gu_rout"]).to(DEV), 2, dcode(c["dn_code"]),
            torch.from_numpy(c["dn_rin"]).to(DEV), torch.from_numpy(c["dn_rout"]).to(DEV), 2)
    ws = torch.zeros(o.moe_expert_path_workspace(1, k, E, H, I), dtype=torch.uint8, device=DEV)
    good = bits16(o.moe_expert_path(*args, ws=ws, one_launch=True))
    assert not np.isnan(good.view(np.float16)).any()
    for via_status in (False, True):
        o.set_moe_spin_limit(0)
        try:
            bad = o.moe_expert_path(*args, ws=ws, one_launch=True).float().cpu()
        finally:
            o.set_moe_spin_limit(-1)
        assert torch.isnan(bad).any()
        if via_status:
            assert o.moe_status(ws, 1, k, H, I) == 1
        else:
            with pytest.raises(_lib.EschaWaitTimeout, match="bounded wait"):
                o.moe_expert_path(*args, ws=ws, one_launch=True)
        assert np.array_equal(bits16(o.moe_expert_path(*args, ws=ws, one_launch=True)), good)
        assert o.moe_status(ws, 1, k, H, I) == 0


@pytest.mark.parametrize("K_gu,K_dn,I", [(2, 2, 512), (2, 3, 512), (3, 3, 512), (3, 2, 1024)])
def test_moe_layers_one_launch_vs_oracle(K_gu, K_dn, I):
    """Independent token-layers in one launch (throughput mode): every layer's
    output against the oracle, bit-identical across repeated launches (I = 512
    takes the 128-column block down items, I = 1024 the split-K ones)."""
    E, H, k, T, L = 32, 1024, 8, 1, 3
    o = ops()
    cases = [_moe_case(E, H, I, K_gu, K_dn, T, k, 40 + l) for l in range(L)]
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    lays, keep = [], []
    for c in cases:
        ids, sc = o.route_topk(dv(c["logits"]), k)
        lay = {"x": dv(c["x"]), "ids": ids, "scores": sc, "gu_code": dcode(c["gu_code"]),
               "gu_rin": dv(c["gu_rin"]), "gu_rout": dv(c["gu_rout"]), "dn_code": dcode(c["dn_code"]),
               "dn_rin": dv(c["dn_rin"]), "dn_rout": dv(c["dn_rout"]),
               "y": torch.empty((T, H), dtype=torch.float16, device=DEV)}
        lays.append(lay)
    table = o.moe_layers_table(lays, DEV)
    ws = torch.zeros(o.moe_layers_workspace(L, T, k, H, I), dtype=torch.uint8, device=DEV)
    o.moe_expert_path_layers(table, T, k, E, H, I, K_gu, K_dn, ws=ws)
    first = [bits16(l["y"]).copy() for l in lays]
    for c, lay in zip(cases, lays):
        ids_np, sc_np = lay["ids"].cpu().numpy(), lay["scores"].cpu().numpy()
        want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
        got = lay["y"].cpu().numpy().astype(np.float32)
        assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
    for _ in range(3):
        o.moe_expert_path_layers(table, T, k, E, H, I, K_gu, K_dn, ws=ws)
        for f, lay in zip(first, lays):
            assert np.array_equal(bits16(lay["y"]), f)


def test_decode_probe_vs_oracle_and_table_mix_bit_identical():
    """esc_decode_probe (4 wave-steps per wave): every lane's sum of x * w
    over its 256 decoded weights against the oracle's reconstruct of the same
    tiles (float32 tolerance), and every table/hash mix (nt of 8 pairs from
    the LDS table) and prefetch depth bit-identical to the hash-only decode."""
    o = ops()
    o.init()
    steps = 4
    words = o.decode_probe_words(steps, 16)
    rng = np.random.default_rng(21)
    u32 = rng.integers(0, 2**32, size=words, dtype=np.uint64).astype(np.uint32)
    code = torch.from_numpy(u32.view(np.int32)).to(DEV)
    outs = {}
    for nt, pf in [(0, 1), (0, 3)] + [(nt, 2) for nt in (2, 3, 4, 5, 6, 8)]:
        out = torch.full((words // (4 * steps),), float("nan"), dtype=torch.float32, device=DEV)
        o.decode_probe(code, steps, nt, 16, out, pf)
        outs[(nt, pf)] = out.cpu().numpy()
    ref = outs[(0, 1)]
    for key, v in outs.items():
        assert np.array_equal(v.view(np.uint32), ref.view(np.uint32)), key
    # the probe's fixed inputs: word j = f16 pair 0x3C00 ^ 0x10 j in both halves;
    # word xpair_index(r) = 2 (r >> 2) | (r & 1) holds row r (low) and r + 2 (high)
    xw = [(0x3C003C00 ^ (j * 0x00100010)) & 0xFFFFFFFF for j in range(8)]
    x = np.zeros(16)
    for r in (0, 1, 4, 5, 8, 9, 12, 13):
        j = 2 * (r >> 2) | (r & 1)
        x[r] = np.array([xw[j] & 0xFFFF], np.uint16).view(np.float16)[0]
        x[r + 2] = np.array([xw[j] >> 16], np.uint16).view(np.float16)[0]
    # wave g, step k, lane l: tile 16 (steps g + k) + l // 4, quarter l % 4
    n_waves = 16
    n_tiles = n_waves * steps * 16
    w = R.reconstruct(u32[:n_tiles * 16].reshape(1, n_tiles, 16), 16, 16 * n_tiles,
                      2).astype(np.float64)
    got = ref[:n_waves * 64].astype(np.float64)
    for g in range(n_waves):
        for lane in range(64):
            q = lane % 4
            cols = [16 * (16 * (steps * g + k) + lane // 4) + 2 * q + (c & 1) + 8 * (c >> 1)
                    for k in range(steps) for c in range(4)]
            terms = x[:, None] * w[:, cols]
            want = terms.sum()
            assert abs(got[64 * g + lane] - want) <= 2e-5 * np.abs(terms).sum() + 1e-30, (g, lane)


def _layers(o, cases, T, H):
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    lays = []
    for c in cases:
        ids, sc = o.route_topk(dv(c["logits"]), c["ids_k"])
        lays.append({"x": dv(c["x"]), "ids": ids, "scores": sc, "gu_code": dcode(c["gu_code"]),
                     "gu_rin": dv(c["gu_rin"]), "gu_rout": dv(c["gu_rout"]),
                     "dn_code": dcode(c["dn_code"]), "dn_rin": dv(c["dn_rin"]),
                     "dn_rout": dv(c["dn_rout"]),
                     "y": torch.empty((T, H), dtype=torch.float16, device=DEV)})
    return lays


@pytest.mark.parametrize("E,H,I,T,k", [(32, 1024, 1024, 1, 8), (16, 1536, 512, 3, 6),
                                       (24, 512, 2048, 2, 4), (48, 1024, 512, 4, 8)])
def test_moe_layers_table_kernels_shapes(E, H, I, T, k):
    """The table-assisted many-layer kernels (K=2 gate_up and down) away from
    config 3's shape: several tokens per layer (the slot combine over top_k
    rows, top_k not a multiple of 8), H = 1536 (12 gate_up items per (row,
    h-block), so a group straddles two workgroups and its hand-off crosses
    XCDs), I = 1024 and 2048 (2 and 4 down input words per lane).  Every
    layer's output against the oracle, bit-identical on repeat calls."""
    L = 3
    o = ops()
    cases = [dict(_moe_case(E, H, I, 2, 2, T, k, 60 + l), ids_k=k) for l in range(L)]
    lays = _layers(o, cases, T, H)
    table = o.moe_layers_table(lays, DEV)
    ws = torch.zeros(o.moe_layers_workspace(L, T, k, H, I), dtype=torch.uint8, device=DEV)
    o.moe_expert_path_layers(table, T, k, E, H, I, 2, 2, ws=ws)
    first = [bits16(l["y"]).copy() for l in lays]
    for c, lay in zip(cases, lays):
        ids_np, sc_np = lay["ids"].cpu().numpy(), lay["scores"].cpu().numpy()
        want = _oracle_moe(c, ids_np, sc_np, E, H, I, 2, 2, np.unique(ids_np)).astype(np.float32)
        got = lay["y"].cpu().numpy().astype(np.float32)
        assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
    for _ in range(2):
        o.moe_expert_path_layers(table, T, k, E, H, I, 2, 2, ws=ws)
        for f, lay in zip(first, lays):
            assert np.array_equal(bits16(lay["y"]), f)


def test_moe_layers_many_layers_grid_beyond_one_workgroup_per_cu():
    """Beyond 8 items per wave on one workgroup per CU the item kernels run
    more workgroups than CUs (each wave's item pointers are staged in LDS):
    132 token-layers cycling 4 routed cases, every layer against its case's
    oracle, then a 4-layer call (one item per wave) on the same workspace,
    then the many-layer call again -- all within tolerance of the oracle, the
    many-layer call repeatable bit-for-bit."""
    E, H, I, k, T, Lc, L = 32, 1024, 512, 8, 1, 4, 132
    o = ops()
    cases = [dict(_moe_case(E, H, I, 2, 2, T, k, 120 + c), ids_k=k) for c in range(Lc)]
    base = _layers(o, cases, T, H)
    want = []
    for c, lay in zip(cases, base):
        ids_np, sc_np = lay["ids"].cpu().numpy(), lay["scores"].cpu().numpy()
        want.append(_oracle_moe(c, ids_np, sc_np, E, H, I, 2, 2, np.unique(ids_np)).astype(np.float32))
    lays = [dict(base[j % Lc], y=torch.empty((T, H), dtype=torch.float16, device=DEV))
            for j in range(L)]
    ws = torch.zeros(o.moe_layers_workspace(L, T, k, H, I), dtype=torch.uint8, device=DEV)
    big, small = o.moe_layers_table(lays, DEV), o.moe_layers_table(base, DEV)

    def check(ls, n):
        for j, lay in enumerate(ls[:n]):
            got = lay["y"].cpu().numpy().astype(np.float32)
            w = want[j % Lc]
            assert np.abs(got - w).max() / np.abs(w).max() < 5e-3, j

    o.moe_expert_path_layers(big, T, k, E, H, I, 2, 2, ws=ws)
    check(lays, L)
    first = [bits16(l["y"]).copy() for l in lays]
    o.moe_expert_path_layers(small, T, k, E, H, I, 2, 2, ws=ws)
    check(base, Lc)
    o.moe_expert_path_layers(big, T, k, E, H, I, 2, 2, ws=ws)
    for f, lay in zip(first, lays):
        assert np.array_equal(bits16(lay["y"]), f)


def test_moe_layers_workspace_shared_by_both_kernel_families():
    """K=2/2 calls run the table-assisted kernels, other K the item kernels;
    alternating them on one workspace stays bit-identical to each on a fresh
    workspace (each family's counters sit where the other writes no floats)."""
    E, H, I, k, T, L = 32, 1024, 512, 8, 1, 2
    o = ops()
    runs = {}
    for kk in ((2, 2), (3, 3)):
        cases = [dict(_moe_case(E, H, I, kk[0], kk[1], T, k, 90 + l), ids_k=k) for l in range(L)]
        lays = _layers(o, cases, T, H)
        runs[kk] = (o.moe_layers_table(lays, DEV), lays)
    nbytes = o.moe_layers_workspace(L, T, k, H, I)
    fresh = {}
    for kk, (table, lays) in runs.items():
        o.moe_expert_path_layers(table, T, k, E, H, I, *kk, ws=torch.zeros(nbytes, dtype=torch.uint8,
                                                                           device=DEV))
        fresh[kk] = [bits16(l["y"]).copy() for l in lays]
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    for kk in ((2, 2), (3, 3), (2, 2), (3, 3), (2, 2)):
        table, lays = runs[kk]
        o.moe_expert_path_layers(table, T, k, E, H, I, *kk, ws=ws)
        for f, lay in zip(fresh[kk], lays):
            assert np.array_equal(bits16(lay["y"]), f), kk


def test_moe_fused_is_deterministic(monkeypatch):
    c = _moe_case(64, 512, 256, 2, 2, 2, 8, 77)
    blk = _block(c, 64, 8, 2, 2, monkeypatch, exact=False)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), 8)
    x = torch.from_numpy(c["x"]).to(DEV)
    first = bits16(blk(x, ids, sc))
    for _ in range(8):
        assert np.array_equal(bits16(blk(x, ids, sc)), first)


def test_moe_config3_shape_fused_vs_exact(monkeypatch):
    """BASELINE config 3 shapes (E=256, H=2048, I=512, top-8, K=2): fused path
    against the order-exact chain, plus the exact chain against the oracle."""
    E, H, I, k = 256, 2048, 512, 8
    c = _moe_case(E, H, I, 2, 2, 1, k, 2)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    y_fast = _block(c, E, k, 2, 2, monkeypatch, False)(x, ids, sc).cpu().numpy().astype(np.float32)
    y_ex = _block(c, E, k, 2, 2, monkeypatch, True)(x, ids, sc).cpu().numpy()
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, 2, 2, np.unique(ids_np)).astype(np.float32)
    assert np.abs(y_ex.astype(np.float32) - want).max() / np.abs(want).max() < 1e-3
    assert np.abs(y_fast - want).max() / np.abs(want).max() < 5e-3


@pytest.mark.parametrize("K_gu,K_dn,T,k", [(2, 3, 2, 8), (3, 2, 3, 4), (2, 2, 1, 10)])
def test_moe_block_down_items_vs_oracle(K_gu, K_dn, T, k, monkeypatch):
    """I == 512, one token-layer: the down leg runs one item per (row,
    128-column block) over all 512 inputs, and the last slot of each (token,
    block) combines the f16 rows in slot order (top_k below, at and above one
    round of 8 slots; 2- and 3-bit codes); repeat calls on one workspace
    agree bit-for-bit (the counters return to zero)."""
    E, H, I = 32, 1024, 512
    c = _moe_case(E, H, I, K_gu, K_dn, T, k, 300 + 10 * K_dn + k)
    blk = _block(c, E, k, K_gu, K_dn, monkeypatch, exact=False)
    ids, sc = ops().route_topk(torch.from_numpy(c["logits"]).to(DEV), k)
    x = torch.from_numpy(c["x"]).to(DEV)
    y = blk(x, ids, sc)
    ids_np, sc_np = ids.cpu().numpy(), sc.cpu().numpy()
    want = _oracle_moe(c, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
    got = y.cpu().numpy().astype(np.float32)
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
    first = bits16(y)
    for _ in range(3):
        assert np.array_equal(bits16(blk(x, ids, sc)), first)


@pytest.mark.parametrize("K_gu,K_dn,k", [(2, 2, 8), (2, 3, 8), (3, 2, 4), (3, 3, 16)])
def test_moe_token_alone_equals_token_in_a_larger_call(K_gu, K_dn, k):
    """I == 512, one token-layer kernels (16-wave gate_up items that decode
    before their inputs arrive, 16-wave down blocks that decode while the
    gate_up partials load): a token routed alone and the same token as token 0
    of a call with more tokens give bit-identical outputs (each row's sums do
    not depend on the other rows), 40 calls in a row on one workspace stay
    bit-identical (the combine counters return to zero), and the output is
    held to the oracle."""
    E, H, I = 64, 2048, 512
    T2 = 16 // k + 1
    c = _moe_case(E, H, I, K_gu, K_dn, T2, k, 500 + 10 * K_gu + K_dn + k)
    o = ops()
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    ids2, sc2 = o.route_topk(dv(c["logits"]), k)
    x2 = dv(c["x"])
    args = (dcode(c["gu_code"]), dv(c["gu_rin"]), dv(c["gu_rout"]), K_gu, dcode(c["dn_code"]),
            dv(c["dn_rin"]), dv(c["dn_rout"]), K_dn)
    y2 = o.moe_expert_path(x2, ids2, sc2, *args)
    x1, ids1, sc1 = x2[:1].contiguous(), ids2[:1].contiguous(), sc2[:1].contiguous()
    ws = torch.zeros(o.moe_expert_path_workspace(1, k, E, H, I), dtype=torch.uint8, device=DEV)
    y1 = o.moe_expert_path(x1, ids1, sc1, *args, ws=ws)
    assert np.array_equal(bits16(y1), bits16(y2[:1]))
    first = bits16(y1)
    for _ in range(40):
        assert np.array_equal(bits16(o.moe_expert_path(x1, ids1, sc1, *args, ws=ws)), first)
    ids_np, sc_np = ids1.cpu().numpy(), sc1.cpu().numpy()
    c1 = dict(c, x=c["x"][:1])
    want = _oracle_moe(c1, ids_np, sc_np, E, H, I, K_gu, K_dn, np.unique(ids_np)).astype(np.float32)
    got = y1.cpu().numpy().astype(np.float32)
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3


# ---------------------------------------------------------------- dense module

def test_dense_linear_module_vs_deploy_and_oracle(dense_linear_golden, monkeypatch):
    from escha_mlx_amd import dense
    monkeypatch.setenv("ESCHA_MLX_BIAS", "1")
    g = dense_linear_golden
    lin = dense.build({"escha_code": g["code"], "escha_rin": g["rin"], "escha_rout": g["rout"],
                       "escha_s_in": g["s_in"], "escha_s_out": g["s_out"], "bias": g["bias"]}, device=DEV)
    y_fast = lin(torch.from_numpy(g["x"]).to(DEV)).cpu().numpy()   # M=8 -> split-K rows (default)
    monkeypatch.setenv("ESCHA_HIP_EXACT", "1")
    lin = dense.build({"escha_code": g["code"], "escha_rin": g["rin"], "escha_rout": g["rout"],
                       "escha_s_in": g["s_in"], "escha_s_out": g["s_out"], "bias": g["bias"]}, device=DEV)
    y = lin(torch.from_numpy(g["x"]).to(DEV)).cpu().numpy()   # M=8 -> fused rows-out, exact order
    rin, rout = R.fold_scales(g["rin"], g["rout"], g["s_in"], g["s_out"])
    want = R.dense_linear(g["x"], g["code"], rin, rout, g["K"], bias=g["bias"], ordered=True)
    assert np.array_equal(y.view(np.uint16), want.view(np.uint16))
    wf = want.astype(np.float32)
    assert np.abs(y_fast.astype(np.float32) - wf).max() <= 2e-3 * np.abs(wf).max()
    monkeypatch.delenv("ESCHA_HIP_EXACT")
    lin = dense.build({"escha_code": g["code"], "escha_rin": g["rin"], "escha_rout": g["rout"],
                       "escha_s_in": g["s_in"], "escha_s_out": g["s_out"], "bias": g["bias"]}, device=DEV)
    dep = g["deploy"].astype(np.float32)
    rel = np.abs(y.astype(np.float32) - dep).mean() / np.abs(dep).mean()
    assert rel < 3e-3
    y1 = lin(torch.from_numpy(g["x"][:1]).to(DEV)).cpu().numpy().astype(np.float32)  # M=1 split-K
    w1 = want[:1].astype(np.float32)
    assert np.abs(y1 - w1).max() <= 2e-3 * np.abs(w1).max()
