"""Write input/output vectors from the reference's own NumPy codec (escha_mlx/ref.py).

Only for the functions that the goldens and closed forms leave open at the bit
level: the H128 butterfly's float32 rounding order, the two transforms, swiglu
(numpy exp), the router softmax, the routed MoE sum in float64, and the full
MoE block (router gate, int8 shared expert, sigmoid gate).  The decode
itself is pinned by the committed goldens and is NOT generated here.

Runs in the build container only (it loads /root/reference/escha_mlx/ref.py by
file path; ref.py depends on numpy alone).  The GPU box and the test suite read
the resulting ``ref_vectors.npz`` and never the reference.

    python tests/golden/make_ref_vectors.py
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

REF = Path("/root/reference/escha_mlx/ref.py")
OUT = Path(__file__).parent / "ref_vectors.npz"


def _load_ref():
    # no bytecode cache: nothing may be written under the read-only reference tree
    sys.dont_write_bytecode = True
    spec = importlib.util.spec_from_file_location("escha_ref_for_vectors", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main() -> None:
    ref = _load_ref()
    rng = np.random.default_rng(20260601)
    v = {}

    # H128 on values whose float32 sums round differently under other orders.
    x = (rng.standard_normal((6, 256)) * np.exp(rng.uniform(-6, 6, (6, 256)))).astype(np.float32)
    v["h128_x"] = x
    v["h128_y"] = ref.h128(x)

    # input transform: f16 rows, signed f32 rin (E-stacked gather done by caller)
    rows = rng.standard_normal((5, 512)).astype(np.float16)
    rin = (rng.choice([-1.0, 1.0], 512) * rng.uniform(0.004, 0.03, 512)).astype(np.float32)
    v["in_x"], v["in_rin"] = rows, rin
    v["in_y"] = ref.input_transform(rows, rin)

    mid = (rng.standard_normal((5, 384)) * 3.0).astype(np.float32)
    rout = (rng.choice([-1.0, 1.0], 384) * rng.uniform(0.5, 1.5, 384) * 1e-2).astype(np.float32)
    v["out_mid"], v["out_rout"] = mid, rout
    v["out_y"] = ref.output_transform(mid, rout)

    gu = (rng.standard_normal((7, 1024)) * 2.0).astype(np.float16)
    v["swiglu_x"] = gu
    v["swiglu_y"] = ref.swiglu(gu)

    # expert linear on a random K=2 stream (tolerance vector: BLAS order)
    code = rng.integers(-32768, 32768, size=(8, 16, 32), dtype=np.int16)
    xl = rng.standard_normal((3, 128)).astype(np.float16)
    rin_l = rng.choice([-1.0, 1.0], 128).astype(np.float32)
    rout_l = (rng.choice([-1.0, 1.0], 256) * rng.uniform(0.5, 1.5, 256) * 1e-2).astype(np.float32)
    v["lin_code"], v["lin_x"], v["lin_rin"], v["lin_rout"] = code, xl, rin_l, rout_l
    v["lin_y"] = ref.expert_linear(xl, code, rin_l, rout_l, 2)

    # routed MoE block (router + experts + shared expert), ids given and routed
    E, H, I, k, T = 8, 128, 128, 2, 3
    w = {
        "gate_w": (rng.standard_normal((E, H)) * 0.1).astype(np.float16),
        "gu_code": rng.integers(-32768, 32768, size=(E, H // 16, 2 * I // 16, 32), dtype=np.int16),
        "gu_rin": rng.choice([-1.0, 1.0], (E, H)).astype(np.float16),
        "gu_rout": (rng.choice([-1.0, 1.0], (E, 2 * I)) * 0.01).astype(np.float16),
        "dn_code": rng.integers(-32768, 32768, size=(E, I // 16, H // 16, 48), dtype=np.int16),
        "dn_rin": rng.choice([-1.0, 1.0], (E, I)).astype(np.float16),
        "dn_rout": (rng.choice([-1.0, 1.0], (E, H)) * 0.01).astype(np.float16),
        "sh_gate_w8": np.zeros((I, H), dtype=np.int8), "sh_gate_scale": np.zeros(I, np.float32),
        "sh_up_w8": np.zeros((I, H), dtype=np.int8), "sh_up_scale": np.zeros(I, np.float32),
        "sh_down_w8": np.zeros((H, I), dtype=np.int8), "sh_down_scale": np.zeros(H, np.float32),
        "shg_w": np.zeros((1, H), dtype=np.float16),
    }
    xm = rng.standard_normal((T, H)).astype(np.float16)
    # zero shared expert: sh*sgate == 0, so the block output is the routed sum
    v["moe_x"] = xm
    v["moe_y"] = ref.moe_block(xm, w, top_k=k)
    logits = (xm.astype(np.float32) @ w["gate_w"].astype(np.float32).T
              ).astype(np.float16).astype(np.float32)
    v["moe_logits"] = logits
    for key in ("gate_w", "gu_code", "gu_rin", "gu_rout", "dn_code", "dn_rin", "dn_rout"):
        v["moe_" + key] = w[key]

    # router on f32 N(0,1) logits (config 3/4 injection: gate Linear bypassed)
    lg = rng.standard_normal((4, 256)).astype(np.float32)
    ids = np.argsort(-lg, axis=-1, kind="stable")[:, :8]
    top = np.take_along_axis(lg, ids, axis=-1)
    e = np.exp(top - top.max(axis=-1, keepdims=True))
    v["route_logits"], v["route_ids"] = lg, ids.astype(np.int32)
    v["route_scores"] = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)

    # full MoE block: router gate, routed experts, a non-zero int8 shared
    # expert and its sigmoid gate (ref.moe_block end to end)
    E, H, I, Ish, k, T = 8, 512, 128, 512, 2, 3
    wb = {
        "gate_w": (rng.standard_normal((E, H)) * 0.05).astype(np.float16),
        "gu_code": rng.integers(-32768, 32768, size=(E, H // 16, 2 * I // 16, 32), dtype=np.int16),
        "gu_rin": rng.choice([-1.0, 1.0], (E, H)).astype(np.float16),
        "gu_rout": (rng.choice([-1.0, 1.0], (E, 2 * I)) * 0.01).astype(np.float16),
        "dn_code": rng.integers(-32768, 32768, size=(E, I // 16, H // 16, 48), dtype=np.int16),
        "dn_rin": rng.choice([-1.0, 1.0], (E, I)).astype(np.float16),
        "dn_rout": (rng.choice([-1.0, 1.0], (E, H)) * 0.01).astype(np.float16),
        "sh_gate_w8": rng.integers(-128, 128, size=(Ish, H), dtype=np.int8),
        "sh_gate_scale": rng.uniform(1e-3, 4e-3, Ish).astype(np.float16).astype(np.float32),
        "sh_up_w8": rng.integers(-128, 128, size=(Ish, H), dtype=np.int8),
        "sh_up_scale": rng.uniform(1e-3, 4e-3, Ish).astype(np.float16).astype(np.float32),
        "sh_down_w8": rng.integers(-128, 128, size=(H, Ish), dtype=np.int8),
        "sh_down_scale": rng.uniform(1e-4, 4e-4, H).astype(np.float16).astype(np.float32),
        "shg_w": (rng.standard_normal((1, H)) * 0.05).astype(np.float16),
    }
    xb = rng.standard_normal((T, H)).astype(np.float16)
    v["blk_x"] = xb
    v["blk_y"] = ref.moe_block(xb, wb, top_k=k)
    for key, val in wb.items():
        v["blk_" + key] = val

    np.savez_compressed(OUT, **v)
    print("wrote", OUT, sorted(v))


if __name__ == "__main__":
    main()
