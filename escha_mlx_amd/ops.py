"""Kernel entry points over torch tensors — the escha_mlx.msl call surface.

Same names, argument meaning and result shapes as the reference's kernel
wrappers (escha_mlx/msl.py); tensors are device tensors on a ROCm GPU and
every call enqueues on torch's current stream.  Code streams are the export's
int16 data viewed as little-endian uint32 words, held in torch as int32
(``code_to_u32``); f16 activations are torch.float16.

Errors: shape / K / row-count preconditions raise ValueError (as the
reference does, escha_mlx/dense.py:170-242, msl.py:1794-1823); a HIP failure
raises EschaHipError.  There is no CPU path: a tensor not on the GPU is an
error.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib, envs

RS = 0.088388347648  # 1/sqrt(128) as pinned by the format (escha_mlx/ref.py:30)


def _ptr(t: torch.Tensor | None):
    # a plain int: every entry point's argtypes convert it (wrapping it in a
    # c_void_p per argument costs more than the launch itself at batch 1)
    return None if t is None else t.data_ptr()


# the current stream's raw handle without building a torch Stream object
# (about 2.9 us per call through torch.cuda.current_stream() on MI355X hosts)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream():
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _dev(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("escha_mlx_amd kernels take GPU tensors (no CPU path)")
        if not t.is_contiguous():
            raise ValueError("escha_mlx_amd kernels take contiguous tensors")


def _as_u32(code: torch.Tensor) -> torch.Tensor:
    if code.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"packed code must be 32-bit words, got {code.dtype}")
    return code


def _lut_flag(lut: bool | None) -> int:
    return int(envs.use_lut() if lut is None else lut)


def code_to_u32(code_i16: np.ndarray) -> np.ndarray:
    """View an int16 code tensor [..., 16K] as little-endian uint32 [..., 8K]
    (escha_mlx/msl.py:1398-1401)."""
    a = np.ascontiguousarray(code_i16).view(np.uint16).astype(np.uint32)
    return (a[..., 0::2] | (a[..., 1::2] << np.uint32(16))).astype(np.uint32)


def to_device_code(code: np.ndarray, device="cuda") -> torch.Tensor:
    """int16 [..., 16K] export (or uint32 [..., 8K]) -> int32 device words."""
    u = code if code.dtype == np.uint32 else code_to_u32(code)
    return torch.from_numpy(np.ascontiguousarray(u).view(np.int32)).to(device)


def init() -> None:
    """Build the decode table on the current device (needed before graph capture)."""
    _lib.call("esc_init")


def decode_tiles(code_u32: torch.Tensor, K: int, IC: int, OC: int,
                 lut: bool | None = None) -> torch.Tensor:
    """One projection's packed stream -> f16 bare weight [IC, OC] (msl.py:1404-1421)."""
    _dev(code_u32)
    code_u32 = _as_u32(code_u32)
    if code_u32.numel() != (IC // 16) * (OC // 16) * 8 * K:
        raise ValueError(f"code has {code_u32.numel()} words, expected a {IC}x{OC} K={K} stream")
    w = torch.empty((IC, OC), dtype=torch.float16, device=code_u32.device)
    _lib.call("esc_decode_tiles", _ptr(code_u32), K, IC, OC, _lut_flag(lut), _ptr(w), _stream())
    return w


# element type codes of esc_input_transform_typed (ESC_ROWS_* in escha_hip.h)
ROWS_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def scaled_had(rows: torch.Tensor, rin: torch.Tensor, row_expert: torch.Tensor | None,
               rs: float = RS) -> torch.Tensor:
    """rows [m, IC] f16, rin [E, IC] f32 (or [IC] with row_expert None) -> [m, IC] f16
    (msl.py:1029-1047, dense variant msl.py:1481-1483).  bf16 and f32 rows are
    transformed from their exact float32 values, with no f16 rounding first, as
    the reference's unfused branch does (dense.py:287-292,
    models/qwen3_5_moe.py:103-110)."""
    _dev(rows, rin, row_expert)
    m, ic = rows.shape
    if rows.dtype not in ROWS_DTYPES:
        raise ValueError(f"rows must be float16, bfloat16 or float32, got {rows.dtype}")
    _check_rows(rows, rows.dtype, rin, row_expert, m, ic)
    if not rows.is_contiguous():
        raise ValueError("rows must be contiguous")
    out = torch.empty((m, ic), dtype=torch.float16, device=rows.device)
    if rows.dtype == torch.float16:
        _lib.call("esc_input_transform", _ptr(rows), _ptr(rin), _ptr(row_expert), m, ic, rs,
                  _ptr(out), _stream())
    else:
        _lib.call("esc_input_transform_typed", _ptr(rows), ROWS_DTYPES[rows.dtype], _ptr(rin),
                  _ptr(row_expert), m, ic, rs, _ptr(out), _stream())
    return out


def as_rows(x2d: torch.Tensor) -> torch.Tensor:
    """Rows for the input transform: f16, bf16 and f32 as they are; any other
    floating type converted to float32 (the reference's rows.astype(float32),
    escha_mlx/dense.py:290); contiguous."""
    if x2d.dtype not in ROWS_DTYPES:
        if not x2d.is_floating_point():
            raise ValueError(f"rows must be floating point, got {x2d.dtype}")
        x2d = x2d.to(torch.float32)
    return x2d.contiguous()


def scaled_had_out(mid: torch.Tensor, rout: torch.Tensor, row_expert: torch.Tensor | None,
                   rs: float = RS, bias: torch.Tensor | None = None) -> torch.Tensor:
    """mid [m, OC] f32, rout [E, OC] f32 (or [OC]) -> f16 [m, OC] (msl.py:1050-1067)."""
    _dev(mid, rout, row_expert, bias)
    m, oc = mid.shape
    _check_rows(mid, torch.float32, rout, row_expert, m, oc)
    out = torch.empty((m, oc), dtype=torch.float16, device=mid.device)
    _lib.call("esc_output_transform", _ptr(mid), _ptr(rout), _ptr(row_expert), _ptr(bias), m, oc,
              rs, _ptr(out), _stream())
    return out


def _check_rows(x, dtype, vec, row_expert, m, dim):
    if x.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {x.dtype}")
    if vec.dtype != torch.float32:
        raise ValueError(f"transform vector must be float32, got {vec.dtype}")
    if row_expert is None:
        if tuple(vec.shape) != (dim,):
            raise ValueError(f"dense transform vector must be ({dim},), got {tuple(vec.shape)}")
    else:
        if vec.dim() != 2 or vec.shape[1] != dim:
            raise ValueError(f"expert transform vectors must be [E, {dim}], got {tuple(vec.shape)}")
        if row_expert.dtype != torch.int32 or tuple(row_expert.shape) != (m,):
            raise ValueError("row_expert must be int32 [m]")


def moe_gemv(xh: torch.Tensor, code_u32: torch.Tensor, row_expert: torch.Tensor | None,
             K: int, IC: int, OC: int, lut: bool | None = None) -> torch.Tensor:
    """mid[r] = xh[r] @ decode(code[row_expert[r]]) in the reference kernel order
    (bit-reproducible; msl.py:1424-1478 with splits=1).  row_expert None = dense."""
    _dev(xh, code_u32, row_expert)
    m = xh.shape[0]
    if xh.dtype != torch.float16 or tuple(xh.shape) != (m, IC):
        raise ValueError(f"xh must be f16 [m, {IC}]")
    mid = torch.empty((m, OC), dtype=torch.float32, device=xh.device)
    _lib.call("esc_gemv", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(row_expert), m, K, IC, OC,
              _lut_flag(lut), _ptr(mid), _stream())
    return mid


def dense_gemv(xh, code_u32, K, IC, OC, lut=None):
    """Dense single-stream GEMV (msl.py:1530-1538)."""
    return moe_gemv(xh, code_u32, None, K, IC, OC, lut)


def gemv_fast_out(xh: torch.Tensor, code_u32: torch.Tensor, row_expert: torch.Tensor | None,
                  rout: torch.Tensor, K: int, IC: int, OC: int, lut: bool | None = None,
                  rs: float = RS) -> torch.Tensor:
    """Split-K GEMV + fused output transform (tolerance contract) -> f16 [m, OC]."""
    _dev(xh, code_u32, row_expert, rout)
    m = xh.shape[0]
    if xh.dtype != torch.float16 or tuple(xh.shape) != (m, IC):
        raise ValueError(f"xh must be f16 [m, {IC}]")
    out = torch.empty((m, OC), dtype=torch.float16, device=xh.device)
    nbytes = _lib.load().esc_gemv_fast_workspace(m, K, IC, OC) if m else 0
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=xh.device)
    _lib.call("esc_gemv_fast_out", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(row_expert),
              _ptr(rout), m, K, IC, OC, _lut_flag(lut), rs, _ptr(out), _ptr(ws), nbytes,
              _stream())
    return out


def moe_gemm_rows(xh: torch.Tensor, code_u32: torch.Tensor, rows_idx: torch.Tensor,
                  group_expert: torch.Tensor, K: int, IC: int, OC: int, R: int, n_rows: int,
                  lut: bool | None = None) -> torch.Tensor:
    """Row-blocked expert GEMM (msl.py:1366-1395).  xh [n_rows+1, IC] with a zero
    row at n_rows; returns mid [n_rows+1, OC] (the caller slices the sink off)."""
    _dev(xh, code_u32, rows_idx, group_expert)
    n_groups = group_expert.shape[0]
    if tuple(xh.shape) != (n_rows + 1, IC):
        raise ValueError(f"xh must be [n_rows+1, {IC}] with a zero sink row")
    if rows_idx.numel() != n_groups * R:
        raise ValueError("rows_idx must hold n_groups*R entries")
    mid = torch.zeros((n_rows + 1, OC), dtype=torch.float32, device=xh.device)
    _lib.call("esc_gemm_rows", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(rows_idx),
              _ptr(group_expert), n_groups, R, n_rows, K, IC, OC, _lut_flag(lut), _ptr(mid),
              _stream())
    return mid


def dense_gemm_rows(xh: torch.Tensor, code_u32: torch.Tensor, K: int, IC: int, OC: int,
                    R: int, lut: bool | None = None) -> torch.Tensor:
    """Dense row-blocked GEMM, bit-identical to dense_gemv (msl.py:1785-1841)."""
    _dev(xh, code_u32)
    m = xh.shape[0]
    mid = torch.empty((m, OC), dtype=torch.float32, device=xh.device)
    _lib.call("esc_dense_gemm_rows", _ptr(xh), _ptr(_as_u32(code_u32)), m, R, K, IC, OC,
              _lut_flag(lut), _ptr(mid), _stream())
    return mid


dense_gemm_rows_direct = dense_gemm_rows


def dense_gemm_rows_direct_out(xh: torch.Tensor, code_u32: torch.Tensor, rout: torch.Tensor,
                               K: int, IC: int, OC: int, R: int, rs: float = RS,
                               lut: bool | None = None) -> torch.Tensor:
    """Dense rows with the fused output transform -> f16 [m, OC] (msl.py:1844-1870)."""
    _dev(xh, code_u32, rout)
    m = xh.shape[0]
    out = torch.empty((m, OC), dtype=torch.float16, device=xh.device)
    _lib.call("esc_dense_gemm_rows_out", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(rout), m, R, K,
              IC, OC, _lut_flag(lut), rs, _ptr(out), _stream())
    return out


LINEAR_SMALL_ROWS = 16


def linear_workspace(m: int, K: int, IC: int, OC: int) -> int:
    return int(_lib.load().esc_linear_workspace(m, K, IC, OC))


def linear(x: torch.Tensor, code_u32: torch.Tensor, rin: torch.Tensor, rout: torch.Tensor, K: int,
           IC: int, OC: int, bias: torch.Tensor | None = None, lut: bool | None = None,
           rs: float = RS, ws: torch.Tensor | None = None) -> torch.Tensor:
    """The whole coded linear (input transform, GEMV/GEMM, output transform,
    optional f16 bias) -> y f16 [m, OC]; one launch below 16 rows
    (dense.py:337-362).  ws must be zero-filled before its first use (the
    one-launch path keeps self-resetting counters there)."""
    _dev(x, code_u32, rin, rout, bias)
    m = x.shape[0]
    if x.dtype != torch.float16 or tuple(x.shape) != (m, IC):
        raise ValueError(f"x must be f16 [m, {IC}]")
    y = torch.empty((m, OC), dtype=torch.float16, device=x.device)
    if m == 0:
        return y
    if ws is None:  # counters (one-launch path) must start at zero; the rest is scratch
        need = linear_workspace(m, K, IC, OC)
        alloc = torch.zeros if m < LINEAR_SMALL_ROWS else torch.empty
        ws = alloc(max(need, 4), dtype=torch.uint8, device=x.device)
    _lib.call("esc_linear", _ptr(x), _ptr(rin), _ptr(_as_u32(code_u32)), _ptr(rout), _ptr(bias), m,
              K, IC, OC, _lut_flag(lut), rs, _ptr(y), _ptr(ws), ws.numel(), _stream())
    return y


def linear_pair_workspace(m: int, K0: int, K1: int, IC: int, OC0: int, OC1: int) -> int:
    return int(_lib.load().esc_linear_pair_workspace(m, K0, K1, IC, OC0, OC1))


def linear_pair(x: torch.Tensor, p0: tuple, p1: tuple, lut: bool | None = None, rs: float = RS,
                ws: torch.Tensor | None = None):
    """Two coded linears over the same rows in one dispatch (dense.py:365-437):
    p0 / p1 = (code_u32, rin, rout, K, OC, bias or None); returns (y0, y1),
    each bit-identical to ``linear`` on its own.  ws must be zero-filled
    before its first use."""
    c0, rin0, rout0, K0, OC0, b0 = p0
    c1, rin1, rout1, K1, OC1, b1 = p1
    _dev(x, c0, rin0, rout0, b0, c1, rin1, rout1, b1)
    m, IC = x.shape
    if x.dtype != torch.float16:
        raise ValueError("x must be float16")
    y0 = torch.empty((m, OC0), dtype=torch.float16, device=x.device)
    y1 = torch.empty((m, OC1), dtype=torch.float16, device=x.device)
    if m == 0:
        return y0, y1
    need = linear_pair_workspace(m, K0, K1, IC, OC0, OC1)
    if ws is None:
        ws = torch.zeros(max(need, 4), dtype=torch.uint8, device=x.device)
    _lib.call("esc_linear_pair", _ptr(x), m, IC, _ptr(rin0), _ptr(_as_u32(c0)), _ptr(rout0),
              _ptr(b0), K0, OC0, _ptr(rin1), _ptr(_as_u32(c1)), _ptr(rout1), _ptr(b1), K1, OC1,
              _lut_flag(lut), rs, _ptr(y0), _ptr(y1), _ptr(ws), ws.numel(), _stream())
    return y0, y1


def _ptr_array(ts) -> ctypes.Array:
    return (ctypes.c_void_p * len(ts))(*[_ptr(t) for t in ts])


def linear_multi_workspace(K: int, IC: int, OCs, m: int = 1) -> int:
    oc = (ctypes.c_int * len(OCs))(*OCs)
    return int(_lib.load().esc_linear_multi_workspace(m, len(OCs), K, IC, oc))


def linear_multi(x: torch.Tensor, projs, lut: bool | None = None, rs: float = RS,
                 ws: torch.Tensor | None = None):
    """1 to 4 coded linears of the same input rows x f16 [m, IC]: projs =
    [(code_u32, rin, rout, K, OC, bias or None), ...] with one K (every OC a
    multiple of 256 at one row).  One row: one launch, each output within the
    tolerance contract of ``linear`` on its own; 2..15 rows: one launch when
    the projections' plans allow, each output bit-identical to ``linear`` on
    its own.  ws must be zero-filled before its first use."""
    _dev(x, *[t for p in projs for t in (p[0], p[1], p[2], p[5])])
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("x must be f16 [m, IC]")
    m, IC = x.shape
    Ks = {p[3] for p in projs}
    if len(Ks) != 1:
        raise ValueError(f"projections with different K {sorted(Ks)}")
    K = Ks.pop()
    OCs = [int(p[4]) for p in projs]
    ys = [torch.empty((m, oc), dtype=torch.float16, device=x.device) for oc in OCs]
    if m == 0:
        return ys
    need = linear_multi_workspace(K, IC, OCs, m)
    if ws is None:
        ws = torch.zeros(max(need, 4), dtype=torch.uint8, device=x.device)
    codes = [_as_u32(p[0]) for p in projs]
    _lib.call("esc_linear_multi", _ptr(x), m, IC, K, len(projs), _ptr_array(codes),
              _ptr_array([p[1] for p in projs]), _ptr_array([p[2] for p in projs]),
              _ptr_array([p[5] for p in projs]), (ctypes.c_int * len(OCs))(*OCs), _lut_flag(lut),
              rs, _ptr_array(ys), _ptr(ws), ws.numel(), _stream())
    return ys


def dense_gemm_rows_fast_out(xh: torch.Tensor, code_u32: torch.Tensor, rout: torch.Tensor,
                             K: int, IC: int, OC: int, R: int, rs: float = RS,
                             lut: bool | None = None) -> torch.Tensor:
    """Dense rows, split-K with R rows per decode + fused output transform ->
    f16 [m, OC] (tolerance contract; msl.py:1844-1870 policy)."""
    _dev(xh, code_u32, rout)
    m = xh.shape[0]
    out = torch.empty((m, OC), dtype=torch.float16, device=xh.device)
    nbytes = _lib.load().esc_gemm_rows_fast_workspace(m, R, K, IC, OC) if m else 0
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=xh.device)
    _lib.call("esc_gemm_rows_fast_out", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(rout), m, R, K,
              IC, OC, _lut_flag(lut), rs, _ptr(out), _ptr(ws), nbytes, _stream())
    return out


def gemm_mfma_out_workspace(m: int, K: int, IC: int, OC: int) -> int:
    return int(_lib.load().esc_gemm_mfma_out_workspace(m, K, IC, OC))


def gemm_mfma_out(xh: torch.Tensor, code_u32: torch.Tensor, rout: torch.Tensor, K: int, IC: int,
                  OC: int, bias: torch.Tensor | None = None, rs: float = RS,
                  ws: torch.Tensor | None = None) -> torch.Tensor:
    """The many-row GEMM with its output transform -> y f16 [m, OC]
    (EschaLinear's dense_gemm_mat + dense_scaled_had_out, dense.py:356): for
    OC a multiple of 256 one launch with the transform in its epilogue, else
    the GEMM into ws (f32 mid) and the output transform."""
    _dev(xh, code_u32, rout, bias)
    m = xh.shape[0]
    if xh.dtype != torch.float16 or tuple(xh.shape) != (m, IC):
        raise ValueError(f"xh must be f16 [m, {IC}]")
    y = torch.empty((m, OC), dtype=torch.float16, device=xh.device)
    if m == 0:
        return y
    if ws is None:
        ws = torch.empty(max(gemm_mfma_out_workspace(m, K, IC, OC), 4), dtype=torch.uint8,
                         device=xh.device)
    _lib.call("esc_gemm_mfma_out", _ptr(xh), _ptr(_as_u32(code_u32)), _ptr(rout), _ptr(bias), m, K,
              IC, OC, rs, _ptr(y), _ptr(ws), ws.numel(), _stream())
    return y


def dense_gemm_mat(xh: torch.Tensor, code_u32: torch.Tensor, K: int, IC: int, OC: int,
                   lut: bool | None = None) -> torch.Tensor:
    """Matrix-core dense GEMM -> mid f32 [m, OC] (msl.py:1762-1782).  Deterministic,
    reassociated float32 sum (tolerance contract); decoded weights bit-exact."""
    _dev(xh, code_u32)
    m = xh.shape[0]
    mid = torch.empty((m, OC), dtype=torch.float32, device=xh.device)
    _lib.call("esc_gemm_mfma", _ptr(xh), _ptr(_as_u32(code_u32)), m, K, IC, OC, _lut_flag(lut),
              _ptr(mid), _stream())
    return mid


def build_groups(row_expert: torch.Tensor, E: int, R: int, n_groups: int):
    """Device sort-and-pack of rows into R-row expert groups (moe.py:30-78)."""
    _dev(row_expert)
    m = row_expert.shape[0]
    rows_idx = torch.empty(n_groups * R, dtype=torch.int32, device=row_expert.device)
    group_expert = torch.empty(n_groups, dtype=torch.int32, device=row_expert.device)
    _lib.call("esc_build_groups", _ptr(row_expert), m, E, R, n_groups, _ptr(rows_idx),
              _ptr(group_expert), _stream())
    return rows_idx, group_expert


def route_topk(logits: torch.Tensor, top_k: int):
    """fp32 logits [T, E] -> ids [T, k] int32, scores [T, k] f32 (ref.py:326-331)."""
    _dev(logits)
    if logits.dtype != torch.float32:
        raise ValueError("router logits must be float32")
    t, e = logits.shape
    ids = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
    scores = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    _lib.call("esc_route_topk", _ptr(logits), t, e, top_k, _ptr(ids), _ptr(scores), _stream())
    return ids, scores


def moe_expert_path_workspace(T: int, top_k: int, E: int, H: int, I: int) -> int:
    return int(_lib.load().esc_moe_expert_path_workspace(T, top_k, E, H, I))


def moe_one_launch_takes(T: int, top_k: int, H: int, I: int) -> bool:
    """Whether esc_moe_expert_path_one_launch takes this shape (up to 64 routed
    rows, top_k <= 32, H a multiple of 256 up to 7936, I a multiple of 128)."""
    return T * top_k <= 64 and top_k <= 32 and H % 256 == 0 and H <= 7936 and I % 128 == 0


def moe_expert_path(x, ids, scores, gu_code, gu_rin, gu_rout, K_gu, dn_code, dn_rin, dn_rout,
                    K_dn, lut=None, ws=None, out=None, one_launch=False):
    """Routed experts for T tokens -> f16 [T, H] (models/qwen3_5_moe.py:207-253).
    one_launch: the whole path as one persistent launch (esc_moe_expert_path_one_launch)
    where the default takes two."""
    _dev(x, ids, scores, gu_code, gu_rin, gu_rout, dn_code, dn_rin, dn_rout)
    t, h = x.shape
    k = ids.shape[1]
    E = gu_code.shape[0]
    I = gu_rout.shape[1] // 2
    if ids.dtype != torch.int32 or scores.dtype != torch.float32:
        raise ValueError("ids must be int32 and scores float32")
    if ws is None:
        # the one-launch path's counters must start at zero; the kernel leaves
        # them zero, so a workspace is reusable for calls of the same shape
        # (a caller's ws is checked against the plan by the library)
        nbytes = moe_expert_path_workspace(t, k, E, h, I)
        ws = torch.zeros(max(nbytes, 4), dtype=torch.uint8, device=x.device)
    y = out if out is not None else torch.empty((t, h), dtype=torch.float16, device=x.device)
    _lib.call("esc_moe_expert_path_one_launch" if one_launch else "esc_moe_expert_path",
              _ptr(x), _ptr(ids), _ptr(scores), t, k, E, h, I,
              _ptr(_as_u32(gu_code)), _ptr(gu_rin), _ptr(gu_rout), K_gu,
              _ptr(_as_u32(dn_code)), _ptr(dn_rin), _ptr(dn_rout), K_dn, _lut_flag(lut),
              _ptr(y), _ptr(ws), ws.numel(), _stream())
    return y


def moe_expert_path_static_max() -> int:
    """Bytes of the device scratch array esc_moe_expert_path_static uses."""
    return int(_lib.load().esc_moe_expert_path_static_max())


def moe_expert_path_static(x, ids, scores, gu_code, gu_rin, gu_rout, K_gu, dn_code, dn_rin,
                           dn_rout, K_dn, out, lut=None):
    """moe_expert_path with no allocation in the call: scratch from the
    library's device array, output into the caller's ``out`` [T, H] f16.
    Calls that overlap on one GPU race (they share the array)."""
    _dev(x, ids, scores, gu_code, gu_rin, gu_rout, dn_code, dn_rin, dn_rout, out)
    t, h = x.shape
    k = ids.shape[1]
    E = gu_code.shape[0]
    I = gu_rout.shape[1] // 2
    if ids.dtype != torch.int32 or scores.dtype != torch.float32:
        raise ValueError("ids must be int32 and scores float32")
    if out.dtype != torch.float16 or tuple(out.shape) != (t, h) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float16 [{t}, {h}] tensor")
    _lib.call("esc_moe_expert_path_static", _ptr(x), _ptr(ids), _ptr(scores), t, k, E, h, I,
              _ptr(_as_u32(gu_code)), _ptr(gu_rin), _ptr(gu_rout), K_gu,
              _ptr(_as_u32(dn_code)), _ptr(dn_rin), _ptr(dn_rout), K_dn, _lut_flag(lut),
              _ptr(out), _stream())
    return out


def decode_probe_words(steps: int, waves_per_cu: int) -> int:
    """Code words esc_decode_probe streams for `steps` wave-steps per wave."""
    return int(_lib.load().esc_decode_probe_words(steps, waves_per_cu))


def decode_probe(code_u32: torch.Tensor, steps: int, nt: int, waves_per_cu: int,
                 out: torch.Tensor, prefetch: int = 1) -> None:
    """Measurement only: the K=2 decode + dot2 loop streamed over `code_u32`
    with nt of every 8 step pairs from the table, `prefetch` wave-steps ahead
    (esc_decode_probe)."""
    _dev(code_u32, out)
    need = decode_probe_words(steps, waves_per_cu)
    lanes = need // (4 * steps) if need else 0  # one output per lane
    if need == 0 or code_u32.numel() < need or out.numel() < lanes:
        raise ValueError(f"probe needs {need} code words and {lanes} outputs")
    _lib.call("esc_decode_probe", _ptr(code_u32), steps, nt, waves_per_cu, prefetch, _ptr(out),
              _stream())


def swiglu(gu16: torch.Tensor) -> torch.Tensor:
    """f16 [m, 2I] -> f16 [m, I]: f16(f16(silu(g)) * u), gate = first half (ref.py:296-301)."""
    _dev(gu16)
    m, two_i = gu16.shape
    h = torch.empty((m, two_i // 2), dtype=torch.float16, device=gu16.device)
    _lib.call("esc_swiglu", _ptr(gu16), m, two_i // 2, _ptr(h), _stream())
    return h


def moe_combine(d16: torch.Tensor, scores: torch.Tensor, top_k: int) -> torch.Tensor:
    """Token-major rows [T*k, H] f16 -> f16 [T, H], weighted slot-order sum
    (models/qwen3_5_moe.py:227-253)."""
    _dev(d16, scores)
    m, h = d16.shape
    t = m // top_k
    y = torch.empty((t, h), dtype=torch.float16, device=d16.device)
    _lib.call("esc_moe_combine", _ptr(d16), _ptr(scores), t, top_k, h, _ptr(y), _stream())
    return y


def w8a16(x: torch.Tensor, w8: torch.Tensor, scale: torch.Tensor,
          out: torch.Tensor | None = None) -> torch.Tensor:
    """x f16 [M, K], w8 int8 [O, K], scale f32 [O] -> f16 [M, O]: the w8a16
    contract wf = f16(f32(w8) * f32(scale)), y = f16(f32-accum x @ wf^T)
    (escha_mlx/quant.py:1-30, ref.py:308-311)."""
    _dev(x, w8, scale)
    if x.dtype != torch.float16 or w8.dtype != torch.int8 or scale.dtype != torch.float32:
        raise ValueError("x must be float16, w8 int8 and scale float32")
    m, k = x.shape
    o = w8.shape[0]
    if w8.shape != (o, k) or scale.shape != (o,):
        raise ValueError(f"shapes x {tuple(x.shape)}, w8 {tuple(w8.shape)}, scale {tuple(scale.shape)}")
    y = out if out is not None else torch.empty((m, o), dtype=torch.float16, device=x.device)
    _lib.call("esc_w8a16", _ptr(x), _ptr(w8), _ptr(scale), m, k, o, _ptr(y), _stream())
    return y


def gemv_f16w(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x f16 [M, K], w f16 [O, K] -> f16 [M, O] = f16(f32-accum x @ w^T): the
    router and shared-expert gates (models/qwen3_5_moe.py:259, 271)."""
    _dev(x, w)
    if x.dtype != torch.float16 or w.dtype != torch.float16:
        raise ValueError("x and w must be float16")
    m, k = x.shape
    o = w.shape[0]
    if w.shape != (o, k):
        raise ValueError(f"shapes x {tuple(x.shape)}, w {tuple(w.shape)}")
    y = out if out is not None else torch.empty((m, o), dtype=torch.float16, device=x.device)
    _lib.call("esc_gemv_f16w", _ptr(x), _ptr(w), m, k, o, _ptr(y), _stream())
    return y


def moe_shared_act(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """f16 [m, I] gate and up -> f16((g / (1 + exp(-g))) * u) (ref.py:345)."""
    _dev(g, u)
    m, i = g.shape
    hh = torch.empty_like(g)
    _lib.call("esc_moe_shared_act", _ptr(g), _ptr(u), m, i, _ptr(hh), _stream())
    return hh


def moe_block_out(y: torch.Tensor, sh: torch.Tensor, shg: torch.Tensor) -> torch.Tensor:
    """f16(f32(y) + f32(sh) * sigmoid(f32(shg))) (models/qwen3_5_moe.py:270-272);
    y, sh f16 [m, H], shg f16 [m, 1] or [m]."""
    _dev(y, sh, shg)
    m, h = y.shape
    out = torch.empty_like(y)
    _lib.call("esc_moe_block_out", _ptr(y), _ptr(sh), _ptr(shg.contiguous()), m, h, _ptr(out),
              _stream())
    return out


def q8_embed(ids: torch.Tensor, w8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """ids int [...], w8 int8 [N, K], scale f32 [N] -> f16 [..., K], the rows
    f16(f32(w8[id]) * f32(scale[id])) (escha_mlx/quant.py:253-266).  An id
    outside [0, N) gives a row of NaN."""
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    _dev(flat, w8, scale)
    if w8.dtype != torch.int8 or scale.dtype != torch.float32 or w8.ndim != 2:
        raise ValueError("w8 must be int8 [N, K] and scale float32 [N]")
    n, k = w8.shape
    if scale.shape != (n,):
        raise ValueError(f"scale shape {tuple(scale.shape)} does not match w8 {tuple(w8.shape)}")
    out = torch.empty((flat.shape[0], k), dtype=torch.float16, device=w8.device)
    _lib.call("esc_q8_embed", _ptr(flat), flat.shape[0], _ptr(w8), _ptr(scale), n, k, _ptr(out),
              _stream())
    return out.reshape(*ids.shape, k)


def moe_status(ws: torch.Tensor, T: int, top_k: int, H: int, I: int) -> int:
    """1 if a one-launch expert path using ``ws``, or any on this device, hit
    its bounded wait since the flags were last read (reading clears them;
    synchronises)."""
    flag = ctypes.c_int32(0)
    _lib.call("esc_moe_status", _ptr(ws), ws.numel(), T, top_k, H, I, ctypes.byref(flag), _stream())
    return int(flag.value)


def set_moe_spin_limit(polls: int) -> None:
    """Test hook: polls before a wait of the one-launch expert path gives up
    (negative restores the default; 0 gives up at once)."""
    _lib.call("esc_moe_set_spin_limit", int(polls))


# one esc_moe_layer record: x, ids, scores, gu_code, gu_rin, gu_rout,
# dn_code, dn_rin, dn_rout, y (device pointers, in that order)
MOE_LAYER_FIELDS = ("x", "ids", "scores", "gu_code", "gu_rin", "gu_rout", "dn_code", "dn_rin",
                    "dn_rout", "y")


def moe_layers_table(layers: list[dict], device) -> torch.Tensor:
    """Device array of esc_moe_layer records for moe_expert_path_layers."""
    rows = []
    for lay in layers:
        _dev(*(lay[f] for f in MOE_LAYER_FIELDS))
        rows.append([lay[f].data_ptr() for f in MOE_LAYER_FIELDS])
    return torch.tensor(rows, dtype=torch.int64).to(device)


def moe_layers_workspace(L: int, T: int, top_k: int, H: int, I: int) -> int:
    return int(_lib.load().esc_moe_layers_workspace(L, T, top_k, H, I))


def moe_expert_path_layers(table: torch.Tensor, T: int, top_k: int, E: int, H: int, I: int,
                           K_gu: int, K_dn: int, ws: torch.Tensor | None = None) -> None:
    """L independent token-layers of routed experts in one launch; each layer's
    y is written in place (see esc_moe_expert_path_layers)."""
    _dev(table)
    L = table.shape[0]
    if ws is None:
        ws = torch.zeros(max(moe_layers_workspace(L, T, top_k, H, I), 4), dtype=torch.uint8,
                         device=table.device)
    _lib.call("esc_moe_expert_path_layers", _ptr(table), L, T, top_k, E, H, I, K_gu, K_dn,
              _ptr(ws), ws.numel(), _stream())
