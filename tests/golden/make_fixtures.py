"""Copy the reference's committed codec goldens into small fixtures.

Run once in the build container (needs /root/reference; the GPU box never runs
this):   python tests/golden/make_fixtures.py

Data only, no reference code is read or executed: the raw little-endian arrays
under /root/reference/tests/data are copied or digested.

  codec/packed_gu_e0_k2.i16    K=2 expert-0 gate_up stream [128,64,32] int16
  codec/packed_down_e0_k3.i16  K=3 expert-0 down stream   [32,128,48] int16
  codec/expected_*.f16         the decoded weights; kept here as a SHA-256 of
                               the full array plus its first 32 rows, so that a
                               bit-exact full comparison needs no 6 MB copy
  qwen3_5/lin_k{2,3}_*         real 128x128 corners with the reference output
                               shipped for them ("deploy"), copied verbatim
"""
from __future__ import annotations

import hashlib
import json
import shutil
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/tests/data")
DST = Path(__file__).parent

HEAD_ROWS = 32


def main() -> None:
    (DST / "codec").mkdir(exist_ok=True)
    (DST / "qwen3_5").mkdir(exist_ok=True)
    meta = {}
    for packed, expected, shape in (
        ("packed_gu_e0_k2.i16", "expected_gu_e0_k2.f16", (2048, 1024)),
        ("packed_down_e0_k3.i16", "expected_down_e0_k3.f16", (512, 2048)),
    ):
        shutil.copyfile(SRC / "codec" / packed, DST / "codec" / packed)
        exp = np.fromfile(SRC / "codec" / expected, dtype=np.float16).reshape(shape)
        exp[:HEAD_ROWS].tofile(DST / "codec" / (expected + f".head{HEAD_ROWS}"))
        meta[expected] = {
            "shape": list(shape),
            "sha256": hashlib.sha256(exp.tobytes()).hexdigest(),
            "head_rows": HEAD_ROWS,
            "n_zero": int((exp.view(np.uint16) & 0x7FFF == 0).sum()),
        }
    for f in sorted((SRC / "qwen3_5").glob("lin_k*")):
        shutil.copyfile(f, DST / "qwen3_5" / f.name)
    (DST / "codec" / "expected_digests.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(json.dumps(meta, indent=1))


if __name__ == "__main__":
    main()
