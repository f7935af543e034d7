"""Routed-expert toolkit: the escha_mlx.moe call surface plus the expert path.

``EschaExperts`` (E-stacked coded projection), ``build_groups``,
``n_groups_bound`` follow escha_mlx/moe.py:30-105.  ``EschaMoEExperts`` is the
routed part of EschaSparseMoeBlock (escha_mlx/models/qwen3_5_moe.py:97-253):
token-major rows, gate_up leg, swiglu, down leg, f16(score)-weighted
slot-order combine, rounded to f16.  ``route`` is its router step on given
float32 logits (models/qwen3_5_moe.py:257-263, in ref.moe_block's stable
order, escha_mlx/ref.py:326-331).

Two execution paths with the same rounding points:
  * fused (default) — ``esc_moe_expert_path``: decode fused into split-K
    GEMVs, transforms / swiglu / combine fused into their epilogues; GEMV
    sums reassociated (tolerance contract), decode bit-exact.
  * exact (ESCHA_HIP_EXACT=1, and ESCHA_MLX_FUSED_HAD=0) — the reference
    kernel chain with the reference accumulation order (bit-reproducible
    against the oracle), row-blocked by the reference's R policy; every
    transform is its own launch.
"""
from __future__ import annotations

import numpy as np
import torch

from . import envs, ops, quant

RS = ops.RS


def n_groups_bound(m: int, E: int, R: int) -> int:
    """Static upper bound on groups: every expert may waste up to R-1 slots (moe.py:81-83)."""
    return (m + E * (R - 1) + R - 1) // R


def build_groups(row_expert: torch.Tensor, E: int, R: int, n_groups: int):
    """Rows sorted by expert into R-row groups, on the device (moe.py:30-78)."""
    return ops.build_groups(row_expert.to(torch.int32).contiguous(), E, R, n_groups)


class EschaExperts:
    """One projection's E-stacked arrays (moe.py:86-105): code [E, TK, TN, 8K]
    words (int32 storage), rin [E, IC] f32, rout [E, OC] f32."""

    def __init__(self, code_i16: np.ndarray, rin: np.ndarray, rout: np.ndarray,
                 device="cuda") -> None:
        if code_i16.ndim != 4:
            raise ValueError(f"expert code must be [E, TK, TN, 16K], got {code_i16.shape}")
        e, tk, tn, wpt2 = code_i16.shape
        if wpt2 % 16 or wpt2 // 16 not in (2, 3):
            raise ValueError(f"escha code last dim {wpt2} implies an unsupported K")
        self.K = wpt2 // 16
        self.E, self.IC, self.OC = e, tk * 16, tn * 16
        if self.IC % 128 or self.OC % 128:
            raise ValueError(f"expert dimensions must be multiples of 128, got {self.IC}x{self.OC}")
        if np.shape(rin) != (e, self.IC) or np.shape(rout) != (e, self.OC):
            raise ValueError("rin/rout must be [E, IC] / [E, OC]")
        self.code = ops.to_device_code(code_i16, device)
        self.rin = torch.from_numpy(np.asarray(rin).astype(np.float32)).to(device)
        self.rout = torch.from_numpy(np.asarray(rout).astype(np.float32)).to(device)

    @classmethod
    def from_device(cls, code: torch.Tensor, rin: torch.Tensor, rout: torch.Tensor, K: int):
        self = cls.__new__(cls)
        self.K = K
        self.E, tk, tn, _ = code.shape
        self.IC, self.OC = tk * 16, tn * 16
        self.code, self.rin, self.rout = code, rin, rout
        return self

    def arrays(self) -> list[torch.Tensor]:
        return [self.code, self.rin, self.rout]


def route(logits: torch.Tensor, top_k: int):
    """float32 logits [T, E] -> (ids [T, k] int32, scores [T, k] float32)."""
    return ops.route_topk(logits.to(torch.float32).contiguous(), top_k)


def blocked_R(m: int, pin: int | None = None) -> int:
    """Rows per expert group for the row-blocked GEMM, 1 = per-row GEMV
    (models/qwen3_5_moe.py:124-170)."""
    if pin is not None:
        return pin
    if m >= 2048:
        return 12
    if m >= 1024:
        return 4
    if m >= 320:
        return 3
    if m >= 128:
        return 2
    return 1


class EschaMoEExperts(torch.nn.Module):
    """Routed experts of one MoE layer: forward(x [T, H] f16, ids [T, k], scores [T, k])
    -> routed sum f16 [T, H] (models/qwen3_5_moe.py:207-253)."""

    def __init__(self, gu: EschaExperts, dn: EschaExperts, num_experts: int, top_k: int) -> None:
        super().__init__()
        if gu.OC != 2 * dn.IC or dn.OC != gu.IC:
            raise ValueError("gate_up [H -> 2I] and down [I -> H] shapes disagree")
        self._gu, self._dn = gu, dn
        self.num_experts, self.top_k = num_experts, top_k
        self._inter = dn.IC
        self._lut = envs.use_lut()
        self._exact = envs.use_exact()
        self._one_launch = envs.moe_one_launch()
        self._fused_had = envs.fused_had()
        self._block_r = envs.block_r_pin()
        envs.kt_block()  # validated like the reference's; no code tiles are staged here
        self._ws = {}

    def _rows(self, t: int, ids: torch.Tensor):
        """Token-major rows: slot s of token t is row t*k + s (qwen3_5_moe.py:97-101)."""
        row_expert = ids.reshape(t * self.top_k).to(torch.int32).contiguous()
        row_token = torch.arange(t, device=ids.device, dtype=torch.int64).repeat_interleave(self.top_k)
        return row_expert, row_token

    def _gemv(self, xh, row_expert, ex: EschaExperts):
        m = xh.shape[0]
        r = blocked_R(m, self._block_r)
        if r == 1:
            return ops.moe_gemv(xh, ex.code, row_expert, ex.K, ex.IC, ex.OC, lut=self._lut)
        ng = n_groups_bound(m, self.num_experts, r)
        rows_idx, group_expert = build_groups(row_expert, self.num_experts, r, ng)
        xh_pad = torch.cat([xh, torch.zeros((1, xh.shape[1]), dtype=xh.dtype, device=xh.device)])
        mid = ops.moe_gemm_rows(xh_pad, ex.code, rows_idx, group_expert, ex.K, ex.IC, ex.OC, r,
                                m, lut=self._lut)
        return mid[:m].contiguous()

    def _forward_staged(self, x, ids, scores, exact: bool = True):
        """The chain as separate launches: input transform, GEMV, output
        transform, SwiGLU, down input transform, GEMV, output transform,
        combine (models/qwen3_5_moe.py:207-253).  exact: the order-exact
        GEMVs (bit-reproducible); otherwise split-K GEMVs with the output
        transform fused (tolerance contract).  x may be f16, bf16 or f32: the
        first transform reads the rows' exact float32 values."""
        t = x.shape[0]
        row_expert, row_token = self._rows(t, ids)
        gu, dn = self._gu, self._dn
        xh = ops.scaled_had(x[row_token].contiguous(), gu.rin, row_expert)
        if exact:
            gu16 = ops.scaled_had_out(self._gemv(xh, row_expert, gu), gu.rout, row_expert)
        else:
            gu16 = ops.gemv_fast_out(xh, gu.code, row_expert, gu.rout, gu.K, gu.IC, gu.OC,
                                     lut=self._lut)
        h = ops.swiglu(gu16)
        xh2 = ops.scaled_had(h, dn.rin, row_expert)
        if exact:
            d16 = ops.scaled_had_out(self._gemv(xh2, row_expert, dn), dn.rout, row_expert)
        else:
            d16 = ops.gemv_fast_out(xh2, dn.code, row_expert, dn.rout, dn.K, dn.IC, dn.OC,
                                    lut=self._lut)
        return ops.moe_combine(d16, scores.reshape(-1).contiguous(), self.top_k)

    def forward(self, x: torch.Tensor, ids: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
        """y f16 [T, H], the routed sum rounded to f16 (models/qwen3_5_moe.py:253).
        x f16 takes the fused expert path; bf16 / f32 rows are transformed from
        their float32 values (models/qwen3_5_moe.py:103-110), then the staged
        chain runs."""
        x = ops.as_rows(x)
        ids = ids.to(torch.int32).contiguous()
        scores = scores.to(torch.float32).contiguous()
        if x.dtype != torch.float16:
            return self._forward_staged(x, ids, scores, exact=self._exact)
        if self._exact or not self._fused_had:
            # ESCHA_MLX_FUSED_HAD off: every transform is its own launch around
            # the GEMVs (models/qwen3_5_moe.py:103-122), the staged chain
            return self._forward_staged(x, ids, scores)
        t, h = x.shape
        # ESCHA_HIP_MOE_ONE_LAUNCH: one launch wherever that launch takes the shape
        one = self._one_launch and ops.moe_one_launch_takes(t, self.top_k, h, self._inter)
        # one zero-initialised workspace per token count and form: the one-launch
        # path keeps its counters there and leaves them zero after every call,
        # and the two forms lay their counters out differently
        key = (t, x.device, one)
        ws = self._ws.get(key)
        if ws is None:
            need = ops.moe_expert_path_workspace(t, self.top_k, self.num_experts, h, self._inter)
            ws = self._ws[key] = torch.zeros(max(need, 4), dtype=torch.uint8, device=x.device)
        gu, dn = self._gu, self._dn
        return ops.moe_expert_path(x, ids, scores, gu.code, gu.rin, gu.rout, gu.K, dn.code,
                                   dn.rin, dn.rout, dn.K, lut=self._lut, ws=ws, one_launch=one)


class EschaSparseMoeBlock(torch.nn.Module):
    """The whole MoE block (models/qwen3_5_moe.py:60-80, 257-273; ref.moe_block,
    escha_mlx/ref.py:314-349): router gate (f16 Linear) -> top-k softmax ->
    routed experts (f16 sum) -> shared expert (w8a16 gate / up, activation,
    w8a16 down) scaled by sigmoid(shared gate) -> f16.

    Constructor inputs as the reference's: hidden size, expert count, top-k,
    the gate_up / down ``EschaExperts``, the router weight gate_w [E, H] and
    shared gate shg_w [1, H] (f16), and ``shared`` with the shared expert's
    ``{gate,up,down}_w8`` int8 [N, K] and ``{gate,up,down}_scale`` [N].  The
    routed sum is rounded to f16 before the shared expert is added (the
    model's forward contract, models/qwen3_5_moe.py:250-253).
    """

    def __init__(self, hidden_size: int, num_experts: int, top_k: int, gu: EschaExperts,
                 dn: EschaExperts, gate_w, shg_w, shared: dict,
                 group_size: int = quant.DEFAULT_GROUP, device=None) -> None:
        super().__init__()
        device = gu.code.device if device is None else device
        if gu.IC != hidden_size or gu.E != num_experts or dn.E != num_experts:
            raise ValueError(f"experts [{gu.E}] {gu.IC} -> {gu.OC} do not match hidden_size "
                             f"{hidden_size} / num_experts {num_experts}")
        as16 = lambda a: (a if torch.is_tensor(a) else torch.from_numpy(np.asarray(a, np.float16))
                          ).to(device=device, dtype=torch.float16).contiguous()
        self.gate_w, self.shg_w = as16(gate_w), as16(shg_w)
        if tuple(self.gate_w.shape) != (num_experts, hidden_size):
            raise ValueError(f"router gate must be [{num_experts}, {hidden_size}], got "
                             f"{tuple(self.gate_w.shape)}")
        if tuple(self.shg_w.shape) != (1, hidden_size):
            raise ValueError(f"shared expert gate must be [1, {hidden_size}], got "
                             f"{tuple(self.shg_w.shape)}")
        self.experts = EschaMoEExperts(gu, dn, num_experts, top_k)
        self.top_k, self.num_experts = top_k, num_experts
        self.sh_gate = quant.make_linear(shared["gate_w8"], shared["gate_scale"], group_size, device)
        self.sh_up = quant.make_linear(shared["up_w8"], shared["up_scale"], group_size, device)
        self.sh_down = quant.make_linear(shared["down_w8"], shared["down_scale"], group_size, device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """out [.., H] in x's dtype.  The routed experts read bf16 / f32 rows
        unrounded; the router gate and the shared expert (f16 weights, int8
        w8a16: f16 activations) read the rows rounded to f16."""
        shape = x.shape
        rows = ops.as_rows(x.reshape(-1, shape[-1]))
        xf = rows.to(torch.float16).contiguous()
        logits = ops.gemv_f16w(xf, self.gate_w).to(torch.float32)
        ids, scores = route(logits, self.top_k)
        y = self.experts(rows, ids, scores)
        hh = ops.moe_shared_act(self.sh_gate(xf), self.sh_up(xf))
        sh = self.sh_down(hh)
        shg = ops.gemv_f16w(xf, self.shg_w)
        return ops.moe_block_out(y, sh, shg).reshape(shape).to(x.dtype)
