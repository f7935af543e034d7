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
  codec/w8a16_*.sub256         the w8a16 golden (x 8x2048, int8 2048x2048, scale,
                               expected 8x2048) cut to its first 256 output
                               channels (w8 rows, scale, expected columns), plus
                               SHA-256 digests of the full files
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
    sub = 256
    w8 = np.fromfile(SRC / "codec" / "w8a16_w8_2048x2048.i8", dtype=np.int8).reshape(2048, 2048)
    sc = np.fromfile(SRC / "codec" / "w8a16_scale_2048.f32", dtype=np.float32)
    xw = np.fromfile(SRC / "codec" / "w8a16_x_8x2048.f16", dtype=np.float16).reshape(8, 2048)
    ew = np.fromfile(SRC / "codec" / "w8a16_expected_8x2048.f16", dtype=np.float16).reshape(8, 2048)
    w8[:sub].tofile(DST / "codec" / f"w8a16_w8_{sub}x2048.i8")
    sc[:sub].tofile(DST / "codec" / f"w8a16_scale_{sub}.f32")
    xw.tofile(DST / "codec" / "w8a16_x_8x2048.f16")
    np.ascontiguousarray(ew[:, :sub]).tofile(DST / "codec" / f"w8a16_expected_8x{sub}.f16")
    for name, arr in (("w8a16_w8_2048x2048.i8", w8), ("w8a16_scale_2048.f32", sc),
                      ("w8a16_expected_8x2048.f16", ew)):
        meta[name] = {"shape": list(arr.shape), "sha256": hashlib.sha256(arr.tobytes()).hexdigest(),
                      "kept_output_channels": sub}
    for f in sorted((SRC / "qwen3_5").glob("lin_k*")):
        shutil.copyfile(f, DST / "qwen3_5" / f.name)
    (DST / "codec" / "expected_digests.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(json.dumps(meta, indent=1))


if __name__ == "__main__":
    main()
