"""C-ABI library and host logic on the CPU (no GPU compute calls).

Precondition failures return ESC_EINVAL before the library touches HIP, so
they are forced here on a machine without a GPU (failure handling runs on the
CPU).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from escha_mlx_amd import _lib, dense, envs, moe, ops

HEADER = Path(__file__).resolve().parent.parent / "include" / "escha_hip.h"
DUMMY = ctypes.c_void_p(0x1000)  # never dereferenced: the calls fail validation first


def header_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(esc_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = header_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in include/escha_hip.h but not exported"


def test_binding_table_matches_header():
    assert sorted(_lib.SIGNATURES) == header_symbols()


def test_version_and_empty_error():
    lib = _lib.load()
    assert lib.esc_version() == 100
    assert isinstance(lib.esc_last_error(), bytes)


def _rc_msg(fn, *args):
    lib = _lib.load()
    rc = getattr(lib, fn)(*args)
    return rc, lib.esc_last_error().decode()


def test_rejects_unsupported_K():
    rc, msg = _rc_msg("esc_decode_tiles", DUMMY, 4, 128, 128, 0, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "K=4" in msg


@pytest.mark.parametrize("ic,oc", [(100, 128), (128, 144), (0, 128), (256, -128)])
def test_rejects_non_128_multiple(ic, oc):
    rc, msg = _rc_msg("esc_gemv", DUMMY, DUMMY, None, 1, 2, ic, oc, 0, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "multiples of 128" in msg


def test_rejects_null_pointers():
    rc, msg = _rc_msg("esc_gemv", None, DUMMY, None, 1, 2, 128, 128, 0, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "null" in msg


def test_rejects_bad_rows_per_group():
    rc, msg = _rc_msg("esc_dense_gemm_rows", DUMMY, DUMMY, 4, 3, 2, 128, 128, 0, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "R=3" in msg


def test_rejects_small_workspace():
    rc, msg = _rc_msg("esc_gemv_fast_out", DUMMY, DUMMY, None, DUMMY, 1, 2, 2048, 1024, 0,
                      ctypes.c_float(0.1), DUMMY, DUMMY, 16, None)
    assert rc == _lib.ESC_ENOSPACE and "workspace" in msg


def test_rejects_topk_above_experts():
    rc, msg = _rc_msg("esc_route_topk", DUMMY, 1, 4, 8, DUMMY, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "top_k" in msg


def test_rejects_groups_below_bound():
    rc, msg = _rc_msg("esc_build_groups", DUMMY, 64, 16, 4, 3, DUMMY, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "bound" in msg


def test_one_launch_expert_path_rejects_shapes_it_does_not_take():
    # 16 tokens x top-8 = 128 routed rows: above the one-launch path's 64
    args = (DUMMY, DUMMY, DUMMY, 16, 8, 256, 2048, 512, DUMMY, DUMMY, DUMMY, 2, DUMMY, DUMMY, DUMMY,
            2, 0, DUMMY, DUMMY, 1 << 30, None)
    rc, msg = _rc_msg("esc_moe_expert_path_one_launch", *args)
    assert rc == _lib.ESC_EINVAL and "T*top_k <= 64" in msg and "T=16" in msg
    # H = 2176 is not a multiple of 256
    args = (DUMMY, DUMMY, DUMMY, 1, 8, 256, 2176, 512) + args[8:]
    rc, msg = _rc_msg("esc_moe_expert_path_one_launch", *args)
    assert rc == _lib.ESC_EINVAL and "H=2176" in msg


def test_one_launch_shape_rule_matches_the_library():
    # the Python rule the module uses to pick the one-launch form, against the
    # library's own rejection on every side of each bound
    from escha_mlx_amd import ops as o
    for T, k, H, I in [(8, 8, 2048, 512), (9, 8, 2048, 512), (1, 8, 7936 + 256, 512),
                       (1, 8, 2176, 512), (1, 8, 2048, 640), (1, 8, 2048, 576), (1, 33, 2048, 512),
                       (2, 32, 1024, 128)]:
        args = (DUMMY, DUMMY, DUMMY, T, k, 256, H, I, DUMMY, DUMMY, DUMMY, 2, DUMMY, DUMMY,
                DUMMY, 2, 0, DUMMY, DUMMY, 0, None)
        rc, msg = _rc_msg("esc_moe_expert_path_one_launch", *args)
        rejected = rc == _lib.ESC_EINVAL and "one-launch" in msg
        assert rejected == (not o.moe_one_launch_takes(T, k, H, I)), (T, k, H, I, rc, msg)


def test_workspace_sizes_are_positive():
    lib = _lib.load()
    assert lib.esc_gemv_fast_workspace(8, 2, 2048, 1024) > 0
    assert lib.esc_moe_expert_path_workspace(1, 8, 256, 2048, 512) > 0
    assert lib.esc_gemv_fast_workspace(8, 4, 2048, 1024) == 0


def test_gemm_mfma_out_workspace_and_rejections():
    """The fused many-row GEMM needs no workspace when the transform runs in its
    epilogue (OC a multiple of 256), M * OC float32 otherwise; bad shapes size
    to 0 and are rejected before any launch, as is a short workspace."""
    lib = _lib.load()
    assert lib.esc_gemm_mfma_out_workspace(64, 2, 1024, 2048) == 0
    assert lib.esc_gemm_mfma_out_workspace(64, 3, 1024, 640) == 64 * 640 * 4
    assert lib.esc_gemm_mfma_out_workspace(64, 4, 1024, 640) == 0
    assert lib.esc_gemm_mfma_out_workspace(64, 2, 1000, 640) == 0
    args = [DUMMY, DUMMY, DUMMY, None, 64, 2, 1024, 640, ctypes.c_float(0.088), DUMMY, DUMMY,
            64 * 640 * 4, None]
    bad = list(args)
    bad[5] = 4
    rc, msg = _rc_msg("esc_gemm_mfma_out", *bad)
    assert rc == _lib.ESC_EINVAL and "K=4" in msg
    bad = list(args)
    bad[9] = None
    rc, msg = _rc_msg("esc_gemm_mfma_out", *bad)
    assert rc == _lib.ESC_EINVAL and "null" in msg
    bad = list(args)
    bad[11] = 16
    rc, msg = _rc_msg("esc_gemm_mfma_out", *bad)
    assert rc == _lib.ESC_ENOSPACE and "workspace" in msg


def test_linear_multi_workspace_and_rejections():
    """esc_linear_multi's workspace: at one row the persistent kernel's
    counters and partials (every OC a multiple of 256), at several rows each
    projection's esc_linear workspace, 256-byte aligned; bad shapes size to 0
    and are rejected before any launch, as is a short workspace."""
    lib = _lib.load()
    oc = lambda *v: (ctypes.c_int * len(v))(*v)
    al = lambda v: (v + 255) // 256 * 256
    for m in (2, 4, 15, 24):
        want = sum(al(lib.esc_linear_workspace(m, 2, 1024, o)) for o in (384, 1280, 512))
        assert lib.esc_linear_multi_workspace(m, 3, 2, 1024, oc(384, 1280, 512)) == want > 0
    assert lib.esc_linear_multi_workspace(1, 2, 2, 1024, oc(512, 1280)) > 0
    assert lib.esc_linear_multi_workspace(1, 2, 2, 1024, oc(512, 384)) == 0   # one row: OC % 256
    assert lib.esc_linear_multi_workspace(0, 1, 2, 1024, oc(512)) == 0
    assert lib.esc_linear_multi_workspace(4, 5, 2, 1024, oc(512, 512, 512, 512, 512)) == 0
    assert lib.esc_linear_multi_workspace(4, 1, 4, 1024, oc(512)) == 0
    ptrs = lambda n: (ctypes.c_void_p * n)(*([DUMMY] * n))
    need = lib.esc_linear_multi_workspace(4, 2, 2, 1024, oc(384, 1280))
    args = [DUMMY, 4, 1024, 2, 2, ptrs(2), ptrs(2), ptrs(2), None, oc(384, 1280), 0,
            ctypes.c_float(0.088), ptrs(2), DUMMY, need, None]
    bad = list(args)
    bad[1] = 1   # one row: OC = 384 is not a multiple of 256
    rc, msg = _rc_msg("esc_linear_multi", *bad)
    assert rc == _lib.ESC_EINVAL and "multiple of 256" in msg
    bad = list(args)
    bad[4] = 5
    rc, msg = _rc_msg("esc_linear_multi", *bad)
    assert rc == _lib.ESC_EINVAL and "projections" in msg
    bad = list(args)
    bad[14] = need - 1
    rc, msg = _rc_msg("esc_linear_multi", *bad)
    assert rc == _lib.ESC_ENOSPACE and "workspace" in msg


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.ESC_EINVAL, "x")
    with pytest.raises(_lib.EschaHipError):
        _lib.check(_lib.ESC_EHIP, "x")


def test_ops_refuse_cpu_tensors():
    with pytest.raises(ValueError, match="GPU"):
        ops.decode_tiles(torch.zeros(16 * 8, dtype=torch.int32), 2, 128, 128)


def test_code_to_u32_little_endian():
    code = np.array([[0x1234, -0x0001, 0x0000, 0x7FFF]], dtype=np.int16)
    assert ops.code_to_u32(code).tolist() == [[0xFFFF1234, 0x7FFF0000]]


# ---------------------------------------------------------------- host policies

def test_dense_block_r_policy():
    """min(m, 16) snapped down to a power of two (escha_mlx/msl.py:1562-1601)."""
    assert [dense.dense_block_r(m) for m in (1, 2, 3, 4, 5, 8, 9, 16, 17, 2048)] == \
        [1, 2, 2, 4, 4, 8, 8, 16, 16, 16]
    assert dense.dense_block_r(100, pin=4) == 4


def test_moe_blocked_r_policy():
    """models/qwen3_5_moe.py:124-170."""
    assert [moe.blocked_R(m) for m in (8, 64, 127, 128, 256, 320, 1024, 2048)] == \
        [1, 1, 1, 2, 2, 3, 4, 12]


def test_n_groups_bound():
    assert moe.n_groups_bound(256, 256, 2) == (256 + 256 + 1) // 2


def _weight(K=2, ic=128, oc=128, **kw):
    rng = np.random.default_rng(0)
    code = rng.integers(-32768, 32768, size=(ic // 16, oc // 16, 16 * K), dtype=np.int16)
    return dense.EschaWeight(code, np.ones(ic, np.float16), np.ones(oc, np.float16),
                             device="cpu", **kw)


def _linear():
    return dense.EschaLinear(_weight())


def test_weight_infers_K_and_folds_scales():
    w = _weight(K=3, s_in=np.full(128, 0.5, np.float32), s_out=np.full(128, 2.0, np.float32))
    assert w.K == 3 and w.IC == 128 and w.OC == 128
    assert torch.all(w.rin == 0.5) and torch.all(w.rout == 2.0)
    assert w.code.dtype == torch.int32 and tuple(w.code.shape) == (8, 8, 24)


def test_weight_rejects_unsupported_K():
    code = np.zeros((8, 8, 64), np.int16)
    with pytest.raises(ValueError, match="K=4"):
        dense.EschaWeight(code, np.ones(128), np.ones(128), device="cpu")


def test_weight_rejects_non_128():
    code = np.zeros((1, 8, 32), np.int16)
    with pytest.raises(ValueError, match="multiples of 128"):
        dense.EschaWeight(code, np.ones(16), np.ones(128), device="cpu")


def test_weight_rejects_2d_transform_vectors():
    code = np.zeros((8, 8, 32), np.int16)
    with pytest.raises(ValueError, match="1-D"):
        dense.EschaWeight(code, np.ones((1, 128)), np.ones(128), device="cpu")


@pytest.mark.parametrize("cfg,msg", [([16, 2, 2, 1, 128], "fields"),
                                     ([16, 3, 2, 1, 128, 128], "disagrees"),
                                     ([16, 2, 2, 2, 128, 128], "codebook")])
def test_weight_config_guards(cfg, msg):
    with pytest.raises(ValueError, match=msg):
        _weight(K=2, config=np.array(cfg))


def test_weight_scale_shape_guard():
    with pytest.raises(ValueError, match="escha_s_in"):
        _weight(s_in=np.ones((2, 128), np.float32))


def test_env_validation(monkeypatch):
    monkeypatch.setenv("ESCHA_MLX_LUT", "maybe")
    with pytest.raises(ValueError, match="ESCHA_MLX_LUT"):
        envs.use_lut()
    monkeypatch.setenv("ESCHA_MLX_DENSE_BLOCK_R", "3")
    with pytest.raises(ValueError, match="ESCHA_MLX_DENSE_BLOCK_R"):
        envs.dense_block_r_pin()


@pytest.mark.parametrize("raw,want", [("1", True), ("true", True), (" Yes ", True), ("ON", True),
                                      ("0", False), ("False", False), ("no", False),
                                      (" off", False), ("", None)])
@pytest.mark.parametrize("name,fn,default", [
    ("ESCHA_MLX_LUT", envs.use_lut, False), ("ESCHA_MLX_FUSED_HAD", envs.fused_had, True),
    ("ESCHA_HIP_EXACT", envs.use_exact, False), ("ESCHA_MLX_DENSE_MAT", envs.dense_mat, True),
    ("ESCHA_MLX_BIAS", dense.apply_bias, False),
    ("ESCHA_HIP_MOE_ONE_LAUNCH", envs.moe_one_launch, False)])
def test_bool_knobs_take_reference_spellings(monkeypatch, name, fn, default, raw, want):
    """Every boolean knob accepts the reference's spellings, blanks and case
    ignored (escha_mlx/envs.py:89-95); empty means the default."""
    monkeypatch.setenv(name, raw)
    assert fn() is (default if want is None else want)


def test_last_logit_knob_spellings(monkeypatch):
    from escha_mlx_amd import loader
    monkeypatch.setenv("ESCHA_MLX_LAST_LOGIT", "false")
    assert loader.use_last_logit() is False
    monkeypatch.setenv("ESCHA_MLX_LAST_LOGIT", " TRUE ")
    assert loader.use_last_logit() is True
    monkeypatch.setenv("ESCHA_MLX_LAST_LOGIT", "2")
    with pytest.raises(ValueError, match="ESCHA_MLX_LAST_LOGIT"):
        loader.use_last_logit()


@pytest.mark.parametrize("raw", ["1", "2", "4", "8", "16", "32"])
def test_kt_block_accepted(monkeypatch, raw):
    monkeypatch.setenv("ESCHA_MLX_KT_BLOCK", raw)
    assert envs.kt_block() == int(raw)


@pytest.mark.parametrize("raw", ["0", "3", "64", "-4", "four"])
def test_kt_block_rejected(monkeypatch, raw):
    """The reference's rule (escha_mlx/envs.py:117-121): a power of two up to 32."""
    monkeypatch.setenv("ESCHA_MLX_KT_BLOCK", raw)
    with pytest.raises(ValueError, match="ESCHA_MLX_KT_BLOCK"):
        envs.kt_block()


def test_modules_validate_kt_block_and_latch_fused_had(monkeypatch):
    """Both knobs are read when a module is built: KT_BLOCK is validated,
    FUSED_HAD is latched (off routes the forward through separate transform
    launches)."""
    ex = moe.EschaExperts(np.zeros((2, 8, 16, 32), np.int16), np.ones((2, 128)),
                          np.ones((2, 256)), device="cpu")
    dn = moe.EschaExperts(np.zeros((2, 8, 8, 32), np.int16), np.ones((2, 128)),
                          np.ones((2, 128)), device="cpu")
    monkeypatch.setenv("ESCHA_MLX_KT_BLOCK", "5")
    with pytest.raises(ValueError, match="ESCHA_MLX_KT_BLOCK"):
        moe.EschaMoEExperts(ex, dn, 2, 1)
    with pytest.raises(ValueError, match="ESCHA_MLX_KT_BLOCK"):
        _linear()
    monkeypatch.setenv("ESCHA_MLX_KT_BLOCK", "8")
    monkeypatch.setenv("ESCHA_MLX_FUSED_HAD", "off")
    assert moe.EschaMoEExperts(ex, dn, 2, 1)._fused_had is False
    assert _linear()._fused_had is False
    monkeypatch.delenv("ESCHA_MLX_FUSED_HAD")
    assert moe.EschaMoEExperts(ex, dn, 2, 1)._fused_had is True


# atomic read-modify-write calls in the HIP sources
_RMW = re.compile(r"\b(atomic(?:Add|Sub|Or|And|Xor|Max|Min|Exch|CAS|Inc|Dec)\w*|unsafeAtomic\w+|"
                  r"safeAtomic\w+|__hip_atomic_(?:fetch_\w+|exchange|compare_exchange_\w+)|"
                  r"__builtin_amdgcn_\w*atomic\w*|__builtin_amdgcn_\w*fadd\w*|"
                  r"__atomic_\w+)\s*\(")


def test_no_float_atomics_in_kernels():
    """Determinism guard (as the reference's tests/test_moe_determinism.py:138):
    every float sum in the kernels has a fixed order, so no atomic
    read-modify-write may touch a float.  Each RMW call site is listed with its
    integer target; a new one must be added here deliberately, after checking
    that its operand is an integer."""
    allowed = {
        ("basic.hpp", "atomicAdd(&s_cnt[row_expert[r]], 1)"),   # int LDS expert counts
        ("basic.hpp", "atomicAdd(&s_cnt[e], 1)"),
        ("basic.hpp", "atomicOr(&s_mask[row_expert[r] * nw + (r >> 6)], 1ull << (r & 63))"),  # u64 bits
        ("fused.hpp", "__hip_atomic_fetch_add(p, v,"),          # add_publish(int* p, int v)
        ("fused.hpp", "__hip_atomic_compare_exchange_strong(p, &expected, 1,"),  # claim(int* p)
        ("fused.hpp", "atomicOr(p.err, 1)"),                      # int flags
        ("fused.hpp", "atomicOr(p.status, 1)"),
        ("escha_hip.hip", "__atomic_exchange_n(h, 0,"),           # host: int wait flag
    }
    csrc = Path(ops.__file__).resolve().parent / "csrc"
    found = set()
    for f in sorted(csrc.glob("*.hpp")) + sorted(csrc.glob("*.hip")):
        for line in f.read_text().splitlines():
            code = line.split("//", 1)[0]
            for m in _RMW.finditer(code):
                site = code[m.start():].strip()
                hit = [a for a in allowed if a[0] == f.name and site.startswith(a[1])]
                assert hit, f"{f.name}: unlisted atomic read-modify-write: {site}"
                found.add(hit[0])
    assert found == allowed, f"listed atomics no longer present: {allowed - found}"
    # the signatures that make the wrapped atomics integer-only
    fused = (csrc / "fused.hpp").read_text()
    assert "int add_publish(int* p, int v)" in fused and "bool claim(int* p)" in fused


def test_experts_container_validation():
    with pytest.raises(ValueError):
        moe.EschaExperts(np.zeros((2, 8, 8, 64), np.int16), np.ones((2, 128)), np.ones((2, 128)),
                         device="cpu")
    ex = moe.EschaExperts(np.zeros((2, 8, 16, 32), np.int16), np.ones((2, 128)),
                          np.ones((2, 256)), device="cpu")
    assert (ex.E, ex.IC, ex.OC, ex.K) == (2, 128, 256, 2)


@pytest.mark.parametrize("fn,K", [("esc_w8a16", 648), ("esc_w8a16", 112), ("esc_w8a16", 8208),
                                  ("esc_gemv_f16w", 60), ("esc_gemv_f16w", 56),
                                  ("esc_gemv_f16w", 4104)])
def test_dense_gemv_rejects_unsupported_K(fn, K):
    if fn == "esc_w8a16":
        rc, msg = _rc_msg(fn, DUMMY, DUMMY, DUMMY, 1, K, 256, DUMMY, None)
    else:
        rc, msg = _rc_msg(fn, DUMMY, DUMMY, 1, K, 256, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and f"K={K}" in msg


def test_w8a16_rejects_null_and_bad_sizes():
    rc, msg = _rc_msg("esc_w8a16", None, DUMMY, DUMMY, 1, 2048, 256, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "null" in msg
    rc, msg = _rc_msg("esc_w8a16", DUMMY, DUMMY, DUMMY, 1, 2048, 0, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "O=0" in msg


def test_q8_embed_rejects_null_and_bad_sizes():
    rc, msg = _rc_msg("esc_q8_embed", None, 1, DUMMY, DUMMY, 4, 32, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "null" in msg
    rc, msg = _rc_msg("esc_q8_embed", DUMMY, 1, DUMMY, DUMMY, 4, 24, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "K=24" in msg
    rc, msg = _rc_msg("esc_q8_embed", DUMMY, 1, DUMMY, DUMMY, 0, 32, DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "N=0" in msg
    rc, _ = _rc_msg("esc_q8_embed", DUMMY, 0, DUMMY, DUMMY, 4, 32, DUMMY, None)
    assert rc == _lib.ESC_OK  # nothing to launch


def test_linear_pair_rejections_and_workspace():
    lib = _lib.load()
    a = lib.esc_linear_workspace(4, 2, 1024, 384)
    assert lib.esc_linear_pair_workspace(4, 2, 3, 1024, 384, 1280) == \
        ((a + 255) & ~255) + lib.esc_linear_workspace(4, 3, 1024, 1280)
    assert lib.esc_linear_pair_workspace(4, 4, 3, 1024, 384, 1280) == 0
    args = [DUMMY, 4, 1024, DUMMY, DUMMY, DUMMY, None, 2, 384, DUMMY, DUMMY, DUMMY, None, 3, 1280,
            0, 0.088, DUMMY, DUMMY, DUMMY, 1 << 30, None]
    bad = list(args)
    bad[13] = 4
    rc, msg = _rc_msg("esc_linear_pair", *bad)
    assert rc == _lib.ESC_EINVAL and "K=4" in msg
    bad = list(args)
    bad[14] = 1000
    rc, msg = _rc_msg("esc_linear_pair", *bad)
    assert rc == _lib.ESC_EINVAL and "multiples of 128" in msg
    bad = list(args)
    bad[18] = None
    rc, msg = _rc_msg("esc_linear_pair", *bad)
    assert rc == _lib.ESC_EINVAL and "null" in msg
    bad = list(args)
    bad[20] = 16
    rc, msg = _rc_msg("esc_linear_pair", *bad)
    assert rc == _lib.ESC_ENOSPACE and "workspace" in msg


def test_input_transform_typed_rejections():
    """esc_input_transform_typed: an unknown row type, a width that is not a
    multiple of 128 and null pointers are refused before any HIP call; the
    Python wrapper refuses non-float rows."""
    rc, msg = _rc_msg("esc_input_transform_typed", DUMMY, 3, DUMMY, None, 4, 128, ctypes.c_float(1.0),
                      DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "row element type" in msg
    rc, msg = _rc_msg("esc_input_transform_typed", DUMMY, 2, DUMMY, None, 4, 100, ctypes.c_float(1.0),
                      DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "divisible by 128" in msg
    rc, msg = _rc_msg("esc_input_transform_typed", None, 1, DUMMY, None, 4, 128, ctypes.c_float(1.0),
                      DUMMY, None)
    assert rc == _lib.ESC_EINVAL and "null" in msg
    assert ops.ROWS_DTYPES == {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
    with pytest.raises(ValueError, match="floating point"):
        ops.as_rows(torch.zeros((2, 128), dtype=torch.int32))
    assert ops.as_rows(torch.zeros((2, 128), dtype=torch.float64)).dtype == torch.float32
