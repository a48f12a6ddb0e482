"""Deterministic synthetic tensors (ctypes over csrc/synth.c).

Each value depends only on (seed, stream, element index), so CPU tests, GPU tests
and bench.py see identical bytes for the same config.
"""
import ctypes
import os

import numpy as np

from . import formats
from ._native import load_synth

_N_THREADS = max(1, min(16, os.cpu_count() or 1))

# sub-seed streams, one per benchmark configuration role
STREAM = {
    "cfg0_w": 0, "cfg1_x": 1, "metric_w": 2, "metric_x": 3,
    "cfg2_up": 4, "cfg2_down": 5, "cfg2_x_up": 6, "cfg2_x_down": 7,
    "cfg4_x": 8, "decode": 100,
}


def key(seed: int, stream: int) -> int:
    return int(load_synth().bpdq_synth_key(ctypes.c_uint64(seed), ctypes.c_uint64(stream)))


def q4k(rows: int, k: int, k64: int, d_sigma=0.02, dmin_sigma=0.01) -> np.ndarray:
    """Q4_K weight [rows x k] as raw bytes (rows * k/256 blocks of 144 B)."""
    nb = rows * (k // formats.Q4K_ELEMS)
    out = np.empty(nb * formats.Q4K_BYTES, dtype=np.uint8)
    load_synth().bpdq_synth_q4k(out.ctypes.data, nb, ctypes.c_uint64(k64), d_sigma, dmin_sigma, _N_THREADS)
    return out


def q8_0(rows: int, k: int, k64: int, d_sigma=0.005) -> np.ndarray:
    nb = rows * (k // formats.Q8_0_ELEMS)
    out = np.empty(nb * formats.Q8_0_BYTES, dtype=np.uint8)
    load_synth().bpdq_synth_q8_0(out.ctypes.data, nb, ctypes.c_uint64(k64), d_sigma, _N_THREADS)
    return out


def normal_f32(n: int, k64: int, sigma=1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load_synth().bpdq_synth_normal_f32(out.ctypes.data, n, ctypes.c_uint64(k64), sigma, _N_THREADS)
    return out


def random_bytes(n: int, k64: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    load_synth().bpdq_synth_bytes(out.ctypes.data, n, ctypes.c_uint64(k64), _N_THREADS)
    return out
