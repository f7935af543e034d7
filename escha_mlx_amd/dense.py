"""Dense coded linear: the escha_mlx.dense call surface on the HIP engine.

``EschaWeight`` / ``EschaLinear`` / ``build`` / ``pack_code`` /
``coded_bytes`` keep the reference's constructor inputs, validation and
forward contract (escha_mlx/dense.py:145-483):

    xh  = f16( H128(x * rin) * RS )
    mid = xh @ decode(code)                       (f32)
    y   = f16( H128(mid) * RS * rout ) [+ bias]

with rin/rout the folded vectors (rin*s_in, rout*s_out in float32,
escha_mlx/ref.py:242-277).  Kernel choice by row count follows
EschaLinear._gemv (dense.py:300-335): M=1 -> GEMV, R = dense_block_r(M)
rows share one decode, R <= 8 with the output transform fused.
"""
from __future__ import annotations

import numpy as np
import torch

from . import envs, ops

RS = ops.RS
SUPPORTED_K = frozenset({2, 3})
_CONFIG_LEN = 6
_PRODUCTION_CODEBOOK = 1
DENSE_R_MAX = 16
# Row count at which the module switches to the matrix-core GEMM: the size
# policy's R = 16 (the reference gates its matrix kernel the same way,
# escha_mlx/dense.py:316-322).
DENSE_MAT_R = 16


def _check_scale(name: str, vec, expect: int) -> None:
    if vec is None:
        return
    shape = tuple(np.shape(vec))
    if shape != (expect,):
        raise ValueError(f"{name} must have shape ({expect},), got {shape}")


def pack_code(code_i16: np.ndarray, device="cuda") -> torch.Tensor:
    """int16 [TK, TN, 16K] -> int32 words [TK, TN, 8K] on the device (dense.py:145-155)."""
    return ops.to_device_code(code_i16, device)


def fold_scales(rin, rout, s_in=None, s_out=None):
    """float32 products rin*s_in, rout*s_out (escha_mlx/ref.py:242-277)."""
    ri = np.asarray(rin).astype(np.float32)
    ro = np.asarray(rout).astype(np.float32)
    if s_in is not None:
        ri = ri * np.asarray(s_in).astype(np.float32)
    if s_out is not None:
        ro = ro * np.asarray(s_out).astype(np.float32)
    return ri, ro


def apply_bias() -> bool:
    """ESCHA_MLX_BIAS on applies the exported correction (default off, dense.py:107-132)."""
    return envs.parse_bool("ESCHA_MLX_BIAS", False)


def dense_block_r(m: int, pin: int | None = None) -> int:
    """Rows per group: min(m, 16) snapped down to a power of two (msl.py:1562-1601)."""
    if pin is not None:
        return pin
    r = min(m, DENSE_R_MAX)
    while r & (r - 1):
        r &= r - 1
    return max(1, r)


class EschaWeight:
    """One dense linear's coded stream and folded transform vectors (dense.py:158-265)."""

    def __init__(self, code, rin, rout, s_in=None, s_out=None, config=None, device="cuda"):
        if isinstance(code, torch.Tensor):
            tk, tn, wpt = code.shape
            if wpt % 8:
                raise ValueError(f"packed escha code last dim must be 8*K, got {wpt}")
            self.K = wpt // 8
            code_dev = code.to(device)
        else:
            tk, tn, wpt2 = np.shape(code)
            if wpt2 % 16:
                raise ValueError(f"escha code last dim must be 16*K, got {wpt2}")
            self.K = wpt2 // 16
            code_dev = None
        if self.K not in SUPPORTED_K:
            raise ValueError(f"escha code implies K={self.K}; this runtime implements "
                             f"K in {sorted(SUPPORTED_K)}")
        self.IC, self.OC = tk * 16, tn * 16
        if np.shape(rin) != (self.IC,) or np.shape(rout) != (self.OC,):
            raise ValueError(
                f"transform vectors {np.shape(rin)}/{np.shape(rout)} do not match the code "
                f"stream's {self.IC}x{self.OC}; both must be 1-D ({self.IC},)/({self.OC},)")
        if self.IC % 128 or self.OC % 128:
            raise ValueError(f"escha linear dimensions must be multiples of 128, got "
                             f"{self.IC}x{self.OC}")
        if config is not None:
            cfg = [int(v) for v in np.asarray(config).ravel()]
            if len(cfg) != _CONFIG_LEN:
                raise ValueError(f"escha_config has {len(cfg)} fields, expected {_CONFIG_LEN} "
                                 "([L, K, V, codebook_id, in_features, out_features])")
            _, k_cfg, _, cb, ic_cfg, oc_cfg = cfg
            if (k_cfg, ic_cfg, oc_cfg) != (self.K, self.IC, self.OC):
                raise ValueError(f"escha_config {(k_cfg, ic_cfg, oc_cfg)} disagrees with the "
                                 f"code stream {(self.K, self.IC, self.OC)}")
            if cb != _PRODUCTION_CODEBOOK:
                raise ValueError(f"escha_config selects codebook id {cb}; this runtime "
                                 f"implements the production codebook (id {_PRODUCTION_CODEBOOK}) only")
        _check_scale("escha_s_in", s_in, self.IC)
        _check_scale("escha_s_out", s_out, self.OC)
        self.code = code_dev if code_dev is not None else pack_code(np.asarray(code), device)
        ri, ro = fold_scales(rin, rout, s_in, s_out)
        self.rin = torch.from_numpy(ri).to(device)
        self.rout = torch.from_numpy(ro).to(device)

    def arrays(self) -> list[torch.Tensor]:
        return [self.code, self.rin, self.rout]


class EschaLinear(torch.nn.Module):
    """A trellis-coded dense linear, drop-in for nn.Linear (dense.py:268-362)."""

    def __init__(self, w: EschaWeight, bias=None) -> None:
        super().__init__()
        self._w = w
        self.bias = None if bias is None else torch.as_tensor(
            np.asarray(bias, dtype=np.float16)).to(w.code.device)
        # latched at construction, like the reference (dense.py:278-281)
        self._lut = envs.use_lut()
        self._exact = envs.use_exact()
        self._block_r_pin = envs.dense_block_r_pin()
        self._mat = envs.dense_mat()
        self._fused_had = envs.fused_had()
        envs.kt_block()  # validated like the reference's; no code tiles are staged here
        self._ws = {}  # zero-filled one-launch workspaces per (rows, device)
        self._pair_ws = {}  # the same for project_pair with this linear first
        self._multi_ws = {}  # the same for project_many with this linear first

    @property
    def K(self) -> int:
        return self._w.K

    def _linear_ws(self, m: int, device) -> torch.Tensor | None:
        if m >= ops.LINEAR_SMALL_ROWS:
            return None  # no counters: a fresh workspace per call
        key = (m, device)
        if key not in self._ws:
            need = ops.linear_workspace(m, self._w.K, self._w.IC, self._w.OC)
            self._ws[key] = torch.zeros(max(need, 4), dtype=torch.uint8, device=device)
        return self._ws[key]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self._w
        shape = x.shape
        # f16 rows take the fused transforms; bf16 / f32 rows are transformed
        # from their float32 values first (dense.py:287-292), then the same
        # kernels run from xh
        rows = ops.as_rows(x.reshape(-1, shape[-1]))
        m = rows.shape[0]
        if (rows.dtype == torch.float16 and not self._exact and self._block_r_pin is None
                and self._fused_had and (m < ops.LINEAR_SMALL_ROWS or self._mat)):
            # the whole linear in esc_linear (one launch below 16 rows)
            y = ops.linear(rows, w.code, w.rin, w.rout, w.K, w.IC, w.OC, bias=self.bias,
                           lut=self._lut, ws=self._linear_ws(m, rows.device))
            return y.reshape(*shape[:-1], w.OC).to(x.dtype)
        xh = ops.scaled_had(rows, w.rin, None)
        r = dense_block_r(m, self._block_r_pin)
        if self._mat and r == DENSE_MAT_R and self._fused_had and not self._exact:
            # the many-row GEMM with the output transform in its epilogue
            y = ops.gemm_mfma_out(xh, w.code, w.rout, w.K, w.IC, w.OC)
        elif self._mat and r == DENSE_MAT_R:
            y = ops.scaled_had_out(ops.dense_gemm_mat(xh, w.code, w.K, w.IC, w.OC), w.rout, None)
        elif not self._fused_had:
            # ESCHA_MLX_FUSED_HAD off: the output transform is its own launch
            # after the GEMV (escha_mlx/dense.py:287-298, 346-356)
            mid = (ops.dense_gemm_rows(xh, w.code, w.K, w.IC, w.OC, r, lut=self._lut) if r > 1
                   else ops.dense_gemv(xh, w.code, w.K, w.IC, w.OC, lut=self._lut))
            y = ops.scaled_had_out(mid, w.rout, None)
        elif m > 1 and r <= 8 and not self._exact:
            y = ops.dense_gemm_rows_fast_out(xh, w.code, w.rout, w.K, w.IC, w.OC, max(r, 2),
                                             lut=self._lut)
        elif m > 1 and r <= 8:
            y = ops.dense_gemm_rows_direct_out(xh, w.code, w.rout, w.K, w.IC, w.OC, r,
                                               lut=self._lut)
        elif r > 1:
            y = ops.scaled_had_out(ops.dense_gemm_rows(xh, w.code, w.K, w.IC, w.OC, r,
                                                       lut=self._lut), w.rout, None)
        elif self._exact:
            y = ops.scaled_had_out(ops.dense_gemv(xh, w.code, w.K, w.IC, w.OC, lut=self._lut),
                                   w.rout, None)
        else:
            y = ops.gemv_fast_out(xh, w.code, None, w.rout, w.K, w.IC, w.OC, lut=self._lut)
        if self.bias is not None:
            y = (y.float() + self.bias.float()).to(torch.float16)
        return y.reshape(*shape[:-1], w.OC).to(x.dtype)


def project_pair(first: EschaLinear, second: EschaLinear, x: torch.Tensor):
    """Two coded projections of the same input in one dispatch
    (escha_mlx/dense.py:365-437): (first(x), second(x)), each bit-identical
    to its own call.  Pairs that do not share the input width or the latched
    decode mode, or that run the order-exact or pinned-R kernels, take two
    calls, as in the reference.  Unlike the reference, one row is fused too:
    the pair launch runs each projection's own one-launch plan, so nothing
    is traded for the saved launch."""
    w0, w1 = first._w, second._w
    shape = x.shape
    rows = x.reshape(-1, shape[-1]).contiguous()
    m = rows.shape[0]
    compatible = (
        rows.dtype == torch.float16
        and w0.IC == w1.IC == rows.shape[-1]
        and first._lut == second._lut
        and first._fused_had and second._fused_had
        and not (first._exact or second._exact)
        and first._block_r_pin is None and second._block_r_pin is None
        and (m < ops.LINEAR_SMALL_ROWS or (first._mat and second._mat))
    )
    if not compatible:
        return first(x), second(x)
    key = (m, rows.device, id(second))
    ws = first._pair_ws.get(key)
    if ws is None:
        need = ops.linear_pair_workspace(m, w0.K, w1.K, w0.IC, w0.OC, w1.OC)
        ws = first._pair_ws[key] = torch.zeros(max(need, 4), dtype=torch.uint8, device=rows.device)
    y0, y1 = ops.linear_pair(rows, (w0.code, w0.rin, w0.rout, w0.K, w0.OC, first.bias),
                             (w1.code, w1.rin, w1.rout, w1.K, w1.OC, second.bias),
                             lut=first._lut, ws=ws)
    return (y0.reshape(*shape[:-1], w0.OC).to(x.dtype), y1.reshape(*shape[:-1], w1.OC).to(x.dtype))


def project_many(linears, x: torch.Tensor):
    """Several coded projections of the same input (an attention block's q, k
    and v): [lin(x) for lin in linears].  Below 16 rows, with one K, the input
    width, the latched decode mode and the fused transforms in common (and at
    one row every OC a multiple of 256), the 2 to 4 projections run as one
    esc_linear_multi call: at one row one launch, each output within the
    tolerance contract of its own call; at 2..15 rows one launch where the
    plans allow, each output bit-identical to its own call.  Otherwise two
    of them take project_pair and the rest their own calls.  No counterpart
    in the reference, which pairs two projections for several rows
    (escha_mlx/dense.py:365-437)."""
    linears = list(linears)
    shape = x.shape
    rows = x.reshape(-1, shape[-1]).contiguous()
    first = linears[0]
    ws_ = [lin._w for lin in linears]
    m = rows.shape[0]
    compatible = (
        rows.dtype == torch.float16 and 2 <= len(linears) <= 4 and 1 <= m < 16
        and len({w.K for w in ws_}) == 1 and all(w.IC == rows.shape[-1] for w in ws_)
        and (m > 1 or all(w.OC % 256 == 0 for w in ws_))
        and len({lin._lut for lin in linears}) == 1
        and all(lin._fused_had and not lin._exact and lin._block_r_pin is None for lin in linears)
    )
    if not compatible:
        if len(linears) == 2:
            return list(project_pair(linears[0], linears[1], x))
        return [lin(x) for lin in linears]
    key = (rows.device, m, tuple(id(lin) for lin in linears[1:]))
    ws = first._multi_ws.get(key)
    if ws is None:
        need = ops.linear_multi_workspace(ws_[0].K, ws_[0].IC, [w.OC for w in ws_], m)
        ws = first._multi_ws[key] = torch.zeros(max(need, 4), dtype=torch.uint8, device=rows.device)
    ys = ops.linear_multi(rows, [(w.code, w.rin, w.rout, w.K, w.OC, lin.bias)
                                 for w, lin in zip(ws_, linears)], lut=first._lut, ws=ws)
    return [y.reshape(*shape[:-1], w.OC).to(x.dtype) for y, w in zip(ys, ws_)]


class EschaMLP(torch.nn.Module):
    """A dense SwiGLU MLP over coded projections with one dispatch for gate and
    up (the fused MLP of escha_mlx/models/qwen3_5.py:63-87):
    down(f16(silu(gate(x)) * up(x))), the activation in float32 with one f16
    rounding."""

    def __init__(self, gate_proj: EschaLinear, up_proj: EschaLinear,
                 down_proj: EschaLinear) -> None:
        super().__init__()
        if gate_proj._w.OC != up_proj._w.OC or down_proj._w.IC != gate_proj._w.OC:
            raise ValueError("gate/up [IC -> I] and down [I -> OC] shapes disagree")
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        gate, up = project_pair(self.gate_proj, self.up_proj, x)
        g = gate.reshape(-1, gate.shape[-1]).to(torch.float16).contiguous()
        u = up.reshape(-1, up.shape[-1]).to(torch.float16).contiguous()
        h = ops.moe_shared_act(g, u)
        return self.down_proj(h).reshape(*shape[:-1], self.down_proj._w.OC).to(x.dtype)


class EschaKVProjection(torch.nn.Module):
    """k and v of an attention layer in one dispatch (the k/v pair of
    escha_mlx/models/qwen3_5.py:90-170; the attention itself is the caller's):
    forward(x) -> (k_proj(x), v_proj(x))."""

    def __init__(self, k_proj: EschaLinear, v_proj: EschaLinear) -> None:
        super().__init__()
        self.k_proj, self.v_proj = k_proj, v_proj

    def forward(self, x: torch.Tensor):
        return project_pair(self.k_proj, self.v_proj, x)


def build(group: dict, device="cuda") -> EschaLinear:
    """Assemble one linear from its tensors keyed by HF leaf name (dense.py:440-452)."""
    w = EschaWeight(group["escha_code"], group["escha_rin"], group["escha_rout"],
                    group.get("escha_s_in"), group.get("escha_s_out"), group.get("escha_config"),
                    device=device)
    bias = group.get("bias") if apply_bias() else None
    return EschaLinear(w, bias)


def coded_bytes(obj) -> int:
    """Bytes of every coded stream under obj (dense.py:455-483)."""
    total, stack, seen = 0, [obj], set()
    while stack:
        node = stack.pop()
        if id(node) in seen:
            continue
        seen.add(id(node))
        if isinstance(node, EschaLinear):
            total += sum(a.numel() * a.element_size() for a in node._w.arrays())
            continue
        if isinstance(node, torch.nn.Module):
            stack.extend(node.children())
        elif isinstance(node, dict):
            stack.extend(node.values())
        elif isinstance(node, (list, tuple)):
            stack.extend(node)
    return total


LEAVES = frozenset({"escha_code", "escha_rin", "escha_rout", "escha_s_in", "escha_s_out",
                    "escha_config", "bias"})
REQUIRED = frozenset({"escha_code", "escha_rin", "escha_rout"})
