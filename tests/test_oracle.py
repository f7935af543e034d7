"""Pin the NumPy oracle (CPU only): goldens, closed forms, brute force, ref vectors.

Each test checks the oracle against something other than its own formula:
the reference's committed decode goldens, Python-integer closed forms, the
Sylvester matrix, brute-force bit strings, or vectors written by the
reference's own ref.py (tests/golden/make_ref_vectors.py).
"""
from __future__ import annotations

import struct

import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import ref_np as R

from .conftest import moe_block_weights, sha256


# ---------------------------------------------------------------- codebook

def test_lut_matches_python_int_closed_form():
    """Every state decoded with Python ints + IEEE half unpacking, summed exactly,
    rounded once to f16 — independent of the oracle's numpy vector code."""
    want = np.empty(65536, dtype=np.float16)
    for s in range(65536):
        r = ((s * 0xCBAC1FED) & 0xFFFFFFFF & 0x8FFF8FFF) ^ 0x3B603B60
        lo = struct.unpack("<e", struct.pack("<H", r & 0xFFFF))[0]
        hi = struct.unpack("<e", struct.pack("<H", r >> 16))[0]
        want[s] = np.float16(lo + hi)  # exact f64 sum, one RNE rounding
    assert np.array_equal(R.LUT.view(np.uint16), want.view(np.uint16))


def test_lut_value_range_and_zeros():
    v = R.LUT.astype(np.float32)
    assert np.abs(v).max() < 4.0
    assert (v == 0).sum() > 0  # exact zeros occur (the goldens hold 392 of them)


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("which", ["k2", "k3"])
def test_reconstruct_bit_exact_vs_goldens(which, k2_golden, k3_golden):
    packed, meta, head = k2_golden if which == "k2" else k3_golden
    K = 2 if which == "k2" else 3
    ic, oc = meta["shape"]
    w = R.reconstruct(packed, ic, oc, K)
    assert np.array_equal(w[: meta["head_rows"]].view(np.uint16), head.view(np.uint16))
    assert sha256(w) == meta["sha256"], "full decoded golden differs"
    n_zero = int(((w.view(np.uint16) & 0x7FFF) == 0).sum())
    assert n_zero == meta["n_zero"]


@pytest.mark.parametrize("K,ic,oc", [(2, 64, 96), (3, 48, 80)])
def test_reconstruct_tiles_loop_equals_vectorised(K, ic, oc):
    """The literal per-tile loop (the CPU baseline's form) decodes the same
    weights as the golden-pinned vectorised reconstruct, int16 and u32 code."""
    rng = np.random.default_rng(40 + K)
    code = rng.integers(-32768, 32768, size=(ic // 16, oc // 16, 16 * K), dtype=np.int16)
    want = R.reconstruct(code, ic, oc, K)
    assert np.array_equal(R.reconstruct_tiles(code, ic, oc, K).view(np.uint16), want.view(np.uint16))
    u32 = R.code_words(code.reshape(-1, 16 * K)).reshape(ic // 16, oc // 16, 8 * K)
    assert np.array_equal(R.reconstruct_tiles(u32, ic, oc, K).view(np.uint16), want.view(np.uint16))


def _brute_states(words: np.ndarray, K: int) -> np.ndarray:
    """Trellis states from an explicit MSB-first bit string (circular)."""
    bits = "".join(format(int(w), "032b") for w in words)
    n = len(bits)
    out = []
    for t in range(256):
        end = K * (t + 1)
        win = "".join(bits[(end - 16 + i) % n] for i in range(16))
        out.append(int(win, 2))
    return np.array(out, dtype=np.uint16)


@pytest.mark.parametrize("K", [2, 3])
def test_tile_states_brute_force(K):
    rng = np.random.default_rng(11 + K)
    words = rng.integers(0, 2**32, size=(5, 8 * K), dtype=np.uint64).astype(np.uint32)
    got = R.tile_states(words, K)
    for i in range(words.shape[0]):
        assert np.array_equal(got[i], _brute_states(words[i], K))


def test_lane_map_bijection():
    row, col = R.lane_map()
    assert len(set(zip(row.tolist(), col.tolist()))) == 256
    assert row.min() == 0 and row.max() == 15 and col.min() == 0 and col.max() == 15


def test_code_words_little_endian():
    code = np.array([[0x1234, -0x0001, 0x0000, 0x7FFF]], dtype=np.int16)
    w = R.code_words(code)
    assert w.tolist() == [[0xFFFF1234, 0x7FFF0000]]


# ---------------------------------------------------------------- transforms

def test_h128_matches_sylvester_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    H = hadamard(128).astype(np.float64)
    want = (x.astype(np.float64).reshape(4, 2, 128) @ H.T).reshape(4, 256)
    got = R.h128(x)
    assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()


def test_h128_involution():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 384)).astype(np.float32)
    assert np.allclose(R.h128(R.h128(x)) / 128.0, x, atol=1e-4)


def test_h128_bit_exact_vs_reference_vectors(ref_vectors):
    got = R.h128(ref_vectors["h128_x"])
    assert np.array_equal(got.view(np.uint32), ref_vectors["h128_y"].view(np.uint32))


def test_h128_rejects_non_multiple():
    with pytest.raises(ValueError):
        R.h128(np.zeros((1, 100), np.float32))


def test_transforms_bit_exact_vs_reference_vectors(ref_vectors):
    v = ref_vectors
    xi = R.input_transform(v["in_x"], v["in_rin"])
    assert np.array_equal(xi.view(np.uint16), v["in_y"].view(np.uint16))
    yo = R.output_transform(v["out_mid"], v["out_rout"])
    assert np.array_equal(yo.view(np.uint16), v["out_y"].view(np.uint16))


def test_swiglu_vs_reference_vectors(ref_vectors):
    got = R.swiglu(ref_vectors["swiglu_x"])
    want = ref_vectors["swiglu_y"]
    # numpy exp on this host: expect identical bits
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_fold_scales_known_answers():
    """Reference tests/test_dense_linear.py:43-62."""
    rin = np.array([2.0, 4.0], dtype=np.float16)
    rout = np.array([3.0], dtype=np.float16)
    ri, ro = R.fold_scales(rin, rout, np.array([0.5, 0.25], np.float32), np.array([2.0], np.float32))
    assert ri.dtype == np.float32 and ro.dtype == np.float32
    assert ri.tolist() == [1.0, 1.0] and ro.tolist() == [6.0]
    ri, ro = R.fold_scales(rin, rout)
    assert np.array_equal(ri, rin.astype(np.float32)) and np.array_equal(ro, rout.astype(np.float32))


# ---------------------------------------------------------------- GEMV order

def _gemv_scalar_loop(xh, w):
    """Sequential float32 scalar loop in the documented order (tiny shapes)."""
    m, ic = xh.shape
    oc = w.shape[1]
    out = np.zeros((m, oc), np.float32)
    for r in range(m):
        for c in range(oc):
            a = [np.float32(0)] * 4
            for kt in range(ic // 16):
                for p in range(4):
                    for off in (0, 1, 8, 9):
                        i = 16 * kt + 2 * p + off
                        a[p] = np.float32(a[p] + np.float32(xh[r, i]) * np.float32(w[i, c]))
            out[r, c] = np.float32(np.float32(a[0] + a[1]) + np.float32(a[2] + a[3]))
    return out


def test_gemv_ordered_matches_scalar_loop():
    rng = np.random.default_rng(5)
    xh = rng.standard_normal((2, 64)).astype(np.float16)
    w = R.LUT[rng.integers(0, 65536, size=(64, 32))]
    got = R.gemv_ordered(xh, w)
    assert np.array_equal(got.view(np.uint32), _gemv_scalar_loop(xh, w).view(np.uint32))


def test_gemv_ordered_close_to_exact_product():
    rng = np.random.default_rng(6)
    xh = rng.standard_normal((3, 512)).astype(np.float16)
    w = R.LUT[rng.integers(0, 65536, size=(512, 256))]
    got = R.gemv_ordered(xh, w)
    want = R.gemv_f64(xh, w)
    assert np.abs(got - want).max() < 1e-5 * np.abs(want).max() * 512 ** 0.5


def test_gemv_ordered_one_hot_reads_weights_back():
    rng = np.random.default_rng(7)
    w = R.LUT[rng.integers(0, 65536, size=(128, 64))]
    xh = np.zeros((3, 128), np.float16)
    rows = [0, 77, 127]
    for r, i in enumerate(rows):
        xh[r, i] = 1.0
    got = R.gemv_ordered(xh, w)
    for r, i in enumerate(rows):
        assert np.array_equal(got[r], w[i].astype(np.float32))


# ---------------------------------------------------------------- linear / routing / MoE

def test_expert_linear_vs_reference_vector(ref_vectors):
    v = ref_vectors
    got = R.expert_linear(v["lin_x"], v["lin_code"], v["lin_rin"], v["lin_rout"], 2).astype(np.float32)
    want = v["lin_y"].astype(np.float32)
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()
    ordered = R.expert_linear(v["lin_x"], v["lin_code"], v["lin_rin"], v["lin_rout"], 2,
                              ordered=True).astype(np.float32)
    assert np.abs(ordered - want).max() <= 2e-3 * np.abs(want).max()


REL_TOL = 3e-3  # reference tests/test_dense_linear.py:31


def test_dense_linear_vs_shipped_deploy_output(dense_linear_golden):
    """Cross-runtime gate on real coded data (reference tests/test_dense_linear.py:68-78)."""
    g = dense_linear_golden
    rin, rout = R.fold_scales(g["rin"], g["rout"], g["s_in"], g["s_out"])
    for ordered in (False, True):
        y = R.dense_linear(g["x"], g["code"], rin, rout, g["K"], bias=g["bias"], ordered=ordered)
        want = g["deploy"].astype(np.float32)
        got = y.astype(np.float32)
        rel = np.abs(got - want).mean() / np.abs(want).mean()
        assert rel < REL_TOL, rel
        assert np.corrcoef(got.ravel(), want.ravel())[0, 1] > 0.9999


def test_dropping_scales_is_visibly_wrong(dense_linear_golden):
    """Reference tests/test_dense_linear.py:99-118: s_in/s_out must matter."""
    g = dense_linear_golden
    want = g["deploy"].astype(np.float32)
    f = R.dense_linear(g["x"], g["code"], *R.fold_scales(g["rin"], g["rout"], g["s_in"], g["s_out"]),
                       g["K"], bias=g["bias"]).astype(np.float32)
    d = R.dense_linear(g["x"], g["code"], *R.fold_scales(g["rin"], g["rout"]), g["K"],
                       bias=g["bias"]).astype(np.float32)
    rf = np.abs(f - want).mean() / np.abs(want).mean()
    rd = np.abs(d - want).mean() / np.abs(want).mean()
    assert rd > 10 * rf


def test_route_topk_vs_reference_vectors(ref_vectors):
    v = ref_vectors
    ids, sc = R.route_topk(v["route_logits"], 8)
    assert np.array_equal(ids, v["route_ids"])
    assert np.allclose(sc, v["route_scores"], rtol=1e-6, atol=0)


def test_route_topk_ties_prefer_lower_id():
    lg = np.array([[1.0, 3.0, 3.0, 0.5, 3.0]], np.float32)
    ids, sc = R.route_topk(lg, 3)
    assert ids.tolist() == [[1, 2, 4]]
    assert np.allclose(sc, 1 / 3)


def test_moe_routed_vs_reference_moe_block(ref_vectors):
    """ref.moe_block with a zero shared expert == the routed sum (f64 accumulation)."""
    v = ref_vectors
    E = v["moe_gate_w"].shape[0]
    ids, sc = R.route_topk(v["moe_logits"], 2)
    H, I = 128, 128
    gu = {"w": np.stack([R.reconstruct(v["moe_gu_code"][e], H, 2 * I, 2) for e in range(E)]),
          "rin": v["moe_gu_rin"], "rout": v["moe_gu_rout"]}
    dn = {"w": np.stack([R.reconstruct(v["moe_dn_code"][e], I, H, 3) for e in range(E)]),
          "rin": v["moe_dn_rin"], "rout": v["moe_dn_rout"]}
    got = R.moe_routed(v["moe_x"], ids, sc, gu, dn, 2, 3, ordered=False, acc64=True)
    want = v["moe_y"]
    diff = np.abs(got.astype(np.float32) - want.astype(np.float32))
    # same BLAS + same f64 sum on this host: at most one f16 ulp apart
    assert diff.max() <= np.abs(want.astype(np.float32)).max() * 2 ** -10


def _groups_brute(row_expert, E, R_, n_groups):
    """Independent model (reference tests/test_blocked.py:25-48)."""
    m = len(row_expert)
    order = np.argsort(row_expert, kind="stable")
    counts = np.bincount(row_expert, minlength=E)
    padded = ((counts + R_ - 1) // R_) * R_
    dst_start = np.cumsum(padded) - padded
    rows_idx = np.full(n_groups * R_, m, dtype=np.int32)
    group_expert = np.full(n_groups, -1, dtype=np.int32)
    p = 0
    for e in range(E):
        c = counts[e]
        if c == 0:
            continue
        rows_idx[dst_start[e]:dst_start[e] + c] = order[p:p + c]
        group_expert[dst_start[e] // R_: (dst_start[e] + padded[e]) // R_] = e
        p += c
    return rows_idx, group_expert


@pytest.mark.parametrize("m,E,R_", [(64, 16, 4), (2048, 256, 16), (517, 32, 8), (8, 256, 4), (256, 256, 2)])
def test_build_groups_model(m, E, R_):
    rng = np.random.default_rng(0)
    re = rng.integers(0, E, size=m).astype(np.int32)
    ng = R.n_groups_bound(m, E, R_)
    a, b = R.build_groups(re, E, R_, ng)
    ra, rb = _groups_brute(re, E, R_, ng)
    assert np.array_equal(a, ra) and np.array_equal(b, rb)
    real = a[a < m]
    assert sorted(real.tolist()) == list(range(m))
    for g in range(ng):
        blk = a[g * R_:(g + 1) * R_]
        occ = blk[blk < m]
        if len(occ):
            assert (re[occ] == b[g]).all()


def test_w8a16_vs_reference_golden(w8a16_golden):
    """The contract's weights f16(f32(w8) * f32(scale)) through a float32 matmul
    agree with the reference's w8a16 golden to its own bar (reference
    tests/test_mlx_cpu.py:55-65: max |diff| / max |want| < 2e-3); the shipped
    outputs are float32 sums in another order, so a few differ by an ulp."""
    w8, scale, x, want = w8a16_golden
    got = R.w8a16(x, w8, scale).astype(np.float32)
    w = want.astype(np.float32)
    assert np.abs(got - w).max() / np.abs(w).max() < 2e-3
    assert (got != w).mean() < 0.05


def test_w8a16_one_hot_reads_contract_weights(w8a16_golden):
    """x = e_k gives y[:, o] = f16(f32(w8[o, k]) * f32(scale[o])) exactly."""
    w8, scale, _, _ = w8a16_golden
    ks = np.array([0, 7, 1000, 2047])
    x = np.zeros((len(ks), 2048), np.float16)
    x[np.arange(len(ks)), ks] = 1.0
    got = R.w8a16(x, w8, scale)
    for i, k in enumerate(ks):
        want = (np.float32(1.0) * (w8[:, k].astype(np.float32) * scale)).astype(np.float16)
        assert np.array_equal(got[i].view(np.uint16), want.view(np.uint16))


def test_q8_dequant_exact_products():
    """Every int8 value times a spread of scales: f16 scales make w8 * scale
    exact in float32 (8 + 11 significant bits), so the contract weight is the
    exact rational product rounded once to f16; f32 scales round the exact
    product to float32 first (the contract's f32 multiply), then to f16.
    Products of an int8 and a float32 are exact in float64, which makes both
    expectations independent of numpy's float32 multiply."""
    from fractions import Fraction
    w8 = np.arange(-128, 128, dtype=np.int8)[None, :]
    s16 = np.array([1e-3, 3.7e-3, 0.0123, 6.1e-5, 1.0, 0.33], np.float16)
    for sc in s16:
        got = R.q8_dequant(w8, np.array([sc], np.float32))[0]
        want = np.array([np.float16(float(Fraction(int(w)) * Fraction(float(sc))))
                         for w in w8[0]], np.float16)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), sc
    for sc in np.array([1.0000001e-3, 2.345678e-3, 7.777777e-2], np.float32):
        got = R.q8_dequant(w8, np.array([sc], np.float32))[0]
        want = np.array([np.float16(np.float32(float(Fraction(int(w)) * Fraction(float(sc)))))
                         for w in w8[0]], np.float16)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), sc


def test_q8_embed_rows_and_shape():
    rng = np.random.default_rng(4)
    w8 = rng.integers(-128, 128, size=(50, 32), dtype=np.int8)
    scale = rng.uniform(1e-3, 5e-3, 50).astype(np.float16)
    ids = np.array([[3, 49], [0, 3]])
    got = R.q8_embed(ids, w8, scale)
    assert got.shape == (2, 2, 32) and got.dtype == np.float16
    wf = R.q8_dequant(w8, scale)
    assert np.array_equal(got[0, 1], wf[49]) and np.array_equal(got[1, 0], wf[0])
    assert np.array_equal(got[0, 0], got[1, 1])


def test_moe_block_vs_reference_moe_block(ref_vectors):
    """The full block (router gate, routed experts, int8 shared expert, sigmoid
    gate) against ref.moe_block: with its float64 routed sum, within an f16
    ulp; with the model's f16 rounding of the routed sum
    (models/qwen3_5_moe.py:250-253), within the f16 tolerance of that extra
    rounding."""
    v = ref_vectors
    w = moe_block_weights(v)
    want = v["blk_y"].astype(np.float32)
    scale = np.abs(want).max()
    got64 = R.moe_block(v["blk_x"], w, 2, routed_f16=False).astype(np.float32)
    assert np.abs(got64 - want).max() <= scale * 2 ** -10
    got16 = R.moe_block(v["blk_x"], w, 2).astype(np.float32)
    assert np.abs(got16 - want).max() <= scale * 2 ** -8
