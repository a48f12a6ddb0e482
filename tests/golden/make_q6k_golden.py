"""Golden vectors for the Q6_K dequant of inference/llamatov_helpers.py:161-179.

That function exists only in the reference's Python and nothing else pins its
element map, so this script imports it from the reference tree (read-only) and
records its outputs on seeded random blocks plus crafted ones (zero / negative /
subnormal / largest scales, every 6-bit quant value).  Run once in a container
that has the reference; the .npz it writes is what the tests read.

    python tests/golden/make_q6k_golden.py /path/to/reference
"""
import os
import sys
import tempfile

import numpy as np


def blocks():
    rng = np.random.default_rng(20261201)
    n = 96
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    d = (np.abs(rng.normal(0, 0.02, n)).astype(np.float16)).view(np.uint8).reshape(n, 2)
    b[:, 208:210] = d                                          # realistic scales for most blocks
    b[0, 208:210] = np.array([0x00, 0x3C], np.uint8)            # d = 1.0
    b[0, 192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)
    b[1, 208:210] = np.array([0x01, 0x00], np.uint8)            # smallest subnormal d
    b[2, 208:210] = np.array([0xFF, 0x7B], np.uint8)            # 65504
    b[2, 192:208] = np.array([127, -128] * 8, np.int8).view(np.uint8)
    b[3, 208:210] = np.array([0x00, 0x80], np.uint8)            # d = -0.0
    b[4, 208:210] = np.array([0x00, 0xBC], np.uint8)            # d = -1.0
    b[5, :128] = 0xFF
    b[5, 128:192] = 0xFF                                        # every quant = +31
    b[6, :192] = 0                                              # every quant = -32
    return b


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "inference"))
    import llamatov_helpers as H

    b = blocks()
    with tempfile.TemporaryDirectory() as td:
        p = os.path.join(td, "q6k.bin")
        b.tofile(p)
        n = b.shape[0] * 256
        y = H.dequant_q6_k(p, 0, n, (n,)).numpy().astype(np.float32)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q6k.npz")
    np.savez_compressed(out, blocks=b.reshape(-1), dequant_ref_order=y)
    print("wrote", out, b.shape, y.shape)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
