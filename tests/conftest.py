from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).parent / "golden"
CODEC = GOLDEN / "codec"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def digests():
    return json.loads((CODEC / "expected_digests.json").read_text())


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _golden(packed_name, expected_name, shape, digests):
    meta = digests[expected_name]
    packed = np.fromfile(CODEC / packed_name, dtype=np.int16).reshape(shape)
    head = np.fromfile(CODEC / f"{expected_name}.head{meta['head_rows']}",
                       dtype=np.float16).reshape(meta["head_rows"], meta["shape"][1])
    return packed, meta, head


@pytest.fixture(scope="session")
def k2_golden(digests):
    """Reference expert-0 gate_up stream, K=2, 2048x1024 (reference tests/conftest.py:55-59)."""
    return _golden("packed_gu_e0_k2.i16", "expected_gu_e0_k2.f16", (128, 64, 32), digests)


@pytest.fixture(scope="session")
def k3_golden(digests):
    """Reference expert-0 down stream, K=3, 512x2048 (reference tests/conftest.py:62-66)."""
    return _golden("packed_down_e0_k3.i16", "expected_down_e0_k3.f16", (32, 128, 48), digests)


@pytest.fixture(scope="session", params=["k2", "k3"])
def dense_linear_golden(request):
    """Real 128x128 corner of a shipped linear + its shipped output (reference
    tests/conftest.py:78-105)."""
    tag = request.param
    d = GOLDEN / "qwen3_5"

    def rd(sfx, dt, shape):
        return np.fromfile(d / f"lin_{tag}_{sfx}", dtype=dt).reshape(shape)

    K = 2 if tag == "k2" else 3
    return {
        "K": K,
        "code": rd("code.i16", np.int16, (8, 8, 16 * K)),
        "rin": rd("rin.f16", np.float16, (128,)),
        "rout": rd("rout.f16", np.float16, (128,)),
        "s_in": rd("s_in.f32", np.float32, (128,)),
        "s_out": rd("s_out.f32", np.float32, (128,)),
        "bias": rd("bias.f16", np.float16, (128,)),
        "x": rd("x.f16", np.float16, (8, 128)),
        "deploy": rd("deploy.f16", np.float16, (8, 128)),
    }


@pytest.fixture(scope="session")
def ref_vectors():
    with np.load(GOLDEN / "ref_vectors.npz") as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def w8a16_golden(digests):
    """The reference's w8a16 golden (reference tests/data/codec/w8a16_*), cut to
    its first output channels: w8 [n, 2048] int8, scale [n] f32, x [8, 2048]
    f16, expected [8, n] f16."""
    n = digests["w8a16_w8_2048x2048.i8"]["kept_output_channels"]
    w8 = np.fromfile(CODEC / f"w8a16_w8_{n}x2048.i8", dtype=np.int8).reshape(n, 2048)
    scale = np.fromfile(CODEC / f"w8a16_scale_{n}.f32", dtype=np.float32)
    x = np.fromfile(CODEC / "w8a16_x_8x2048.f16", dtype=np.float16).reshape(8, 2048)
    want = np.fromfile(CODEC / f"w8a16_expected_8x{n}.f16", dtype=np.float16).reshape(8, n)
    return w8, scale, x, want


def moe_block_weights(v, prefix="blk_"):
    """The full-block weights of a ref_vectors set as oracle.moe_block takes them."""
    from oracle import ref_np as R
    E, H = v[prefix + "gate_w"].shape
    I = v[prefix + "gu_rout"].shape[1] // 2
    gu = {"w": np.stack([R.reconstruct(v[prefix + "gu_code"][e], H, 2 * I, 2) for e in range(E)]),
          "rin": v[prefix + "gu_rin"], "rout": v[prefix + "gu_rout"]}
    dn = {"w": np.stack([R.reconstruct(v[prefix + "dn_code"][e], I, H, 3) for e in range(E)]),
          "rin": v[prefix + "dn_rin"], "rout": v[prefix + "dn_rout"]}
    w = {"gate_w": v[prefix + "gate_w"], "gu": gu, "dn": dn, "shg_w": v[prefix + "shg_w"]}
    for k in ("sh_gate_w8", "sh_gate_scale", "sh_up_w8", "sh_up_scale", "sh_down_w8",
              "sh_down_scale"):
        w[k] = v[prefix + k]
    return w
