#!/usr/bin/env python3
"""Writes tests/golden/loader_test.hypno: the file that hypno's own loader test
builds in memory (create_test_hypno, loader.rs:224-292), rebuilt byte for byte
from that test's steps:

  header (2 metadata pairs, 2 tensors); pairs architecture=llama and
  hidden_size=64; data start = (bytes so far + the test's table estimate
  2 x (4+10+4+8+4+8+8)) rounded up to 64; tensor "weight" FP32 [64] = 0..63 at
  the data start; tensor "qweight" Q4_0 [32] = one block quantised from
  i * 0.1 (f32) at the next 64-byte boundary; no trailing padding.

The Q4_0 block comes from the oracle's quantize_f32_to_q4_0 restatement
(quant.rs:49-71).  The test's assertions (loader.rs:296-319) are checked in
tests/test_model.py.  Regenerate with `python3 tests/golden/make_hypno_fixture.py`.
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402

ALIGN = 64


def build() -> bytes:
    buf = bytearray(struct.pack("<4sIII", b"HYPN", 1, 2, 2))
    for k, v in (("architecture", "llama"), ("hidden_size", "64")):
        buf += struct.pack("<I", len(k)) + k.encode() + struct.pack("<I", len(v)) + v.encode()
    fp32 = np.arange(64, dtype=np.float32).tobytes()
    q4 = orc.quantize_q4_0(np.arange(32, dtype=np.float32) * np.float32(0.1)).tobytes()
    approx = len(buf) + 2 * (4 + 10 + 4 + 8 + 4 + 8 + 8)
    data_start = (approx + ALIGN - 1) // ALIGN * ALIGN
    q4_off = (data_start + len(fp32) + ALIGN - 1) // ALIGN * ALIGN
    for name, n, dtype, off, payload in (("weight", 64, 0, data_start, fp32),
                                         ("qweight", 32, 3, q4_off, q4)):
        buf += struct.pack("<I", len(name)) + name.encode() + struct.pack("<I", 1)
        buf += struct.pack("<QIQQ", n, dtype, off, len(payload))
    buf += bytes(data_start - len(buf))
    buf += fp32
    buf += bytes(q4_off - len(buf))
    buf += q4
    return bytes(buf)


if __name__ == "__main__":
    out = os.path.join(HERE, "loader_test.hypno")
    data = build()
    with open(out, "wb") as f:
        f.write(data)
    print(f"wrote {out} ({len(data)} bytes)")
