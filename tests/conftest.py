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
