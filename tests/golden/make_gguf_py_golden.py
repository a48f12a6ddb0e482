"""Golden vectors for the reference Python loader's per-type dequant
(inference/llamatov_helpers.py:25-158, dispatched by load_tensor_by_type at :196-222):
F16, Q4_0, Q2_K, Q3_K (the reference's approximate form) and Q4_K.

Those functions exist only in the reference's Python. Nothing else pins their element
maps or their operation order: no reference C exists for them, and no fixture either.
So this script imports them from the reference tree (read-only) and records their outputs.
The inputs are seeded random blocks plus crafted scales: 1.0, -0.0, the smallest
subnormal, 65504, +/-Inf, quiet and signalling NaNs with payloads, and NaN in both d
and dmin. Run it once in a container that has the reference; the .npz it writes is what
the tests read.

    python tests/golden/make_gguf_py_golden.py /path/to/reference
"""
import os
import sys
import tempfile

import numpy as np

# (GGUF type, block bytes, elements per block, byte offsets of the f16 scales)
TYPES = {"q4_0": (2, 18, 32, (0,)), "q2_k": (10, 84, 256, (80, 82)), "q3_k": (11, 110, 256, (108,)),
         "q4_k": (12, 144, 256, (0, 2))}
SPECIAL = [0x3C00, 0x8000, 0x0001, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0xFE01, 0x7C01, 0x7D55, 0xBC00, 0x0400]


def blocks(name, seed):
    _, size, _, offs = TYPES[name]
    rng = np.random.default_rng(seed)
    n = 64
    b = rng.integers(0, 256, (n, size), dtype=np.uint8)
    for o in offs:  # realistic scales for most blocks
        b[:, o:o + 2] = np.abs(rng.normal(0, 0.02, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    for i, h in enumerate(SPECIAL):  # each special value in each scale slot
        for k, o in enumerate(offs):
            r = 2 * i + k
            b[r, o:o + 2] = np.array([h & 0xFF, h >> 8], np.uint8)
    for k, o in enumerate(offs):  # NaN in every scale of one block (which NaN a difference keeps)
        b[40, o:o + 2] = np.array([0x01 + k, 0x7E if k == 0 else 0xFE], np.uint8)
    b[41, :] = 0xFF
    b[42, [o for o in offs]] = 0
    b[42, [o + 1 for o in offs]] = 0x3C
    return b


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "inference"))
    import llamatov_helpers as H

    out = {}
    with tempfile.TemporaryDirectory() as td:
        for seed, (name, (code, size, per, _)) in enumerate(TYPES.items()):
            b = blocks(name, 20261202 + seed)
            p = os.path.join(td, name + ".bin")
            b.tofile(p)
            n = b.shape[0] * per
            y = H.load_tensor_by_type(p, 0, n, (n,), code).numpy().astype(np.float32)
            out[name + "_blocks"] = b.reshape(-1)
            out[name + "_dequant"] = y
        h = np.concatenate([np.array(SPECIAL + [0x7FFF, 0xFFFF, 0x8001, 0x03FF], np.uint16),
                            np.random.default_rng(20261210).integers(0, 65536, 4096, dtype=np.uint16)])
        p = os.path.join(td, "f16.bin")
        h.tofile(p)
        out["f16_bits"] = h
        out["f16_dequant"] = H.load_tensor_by_type(p, 0, h.size, (h.size,), 1).numpy().astype(np.float32)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_py.npz")
    np.savez_compressed(dst, **out)
    print("wrote", dst, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
