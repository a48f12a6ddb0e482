"""The reference Python loader's per-type dequant (load_tensor_by_type,
inference/llamatov_helpers.py:196-222) on the GPU through the C ABI
(bpd_dequant_gguf_py_gpu), bit for bit (NaN bits included):

* against the reference's own outputs on the golden blocks
  (tests/golden/gguf_py.npz);
* against the oracle on large random tensors, at source offsets of 1 byte (2
  for Q6_K), and on F16/F32 lengths that leave a tail of 1-3 elements."""
import os

import numpy as np
import pytest

from bpd_substrate_amd import gpu
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "gguf_py.npz")
TYPES = {"q4_0": 2, "q2_k": 10, "q3_k": 11, "q4_k": 12}


def _d(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _at_offset(raw, off, dev):
    """raw's bytes on the device starting `off` bytes into a fresh allocation."""
    import torch

    buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=dev)
    buf[off:off + raw.size] = _d(raw, dev)
    return buf[off:off + raw.size]


@pytest.mark.parametrize("name", list(TYPES))
def test_golden_blocks(dev, name):
    g = np.load(GOLD)
    raw, want = g[name + "_blocks"], g[name + "_dequant"]
    got = gpu.dequant_gguf_py(_d(raw, dev), want.size, TYPES[name])
    assert_bits_equal(to_np(got), want, f"{name} golden")


def test_golden_f16(dev):
    g = np.load(GOLD)
    h, want = g["f16_bits"], g["f16_dequant"]
    got = gpu.dequant_gguf_py(_d(h.view(np.uint8), dev), h.size, 1)
    assert_bits_equal(to_np(got), want, "f16 golden")


@pytest.mark.parametrize("code", [2, 10, 11, 12, 14])
@pytest.mark.parametrize("off", [0, 1])
def test_random_tensors_any_offset(dev, code, off):
    per, size = gpu.GGUF_PY_BLOCKS[code]
    off = 2 * off if code == 14 else off  # Q6_K: 2-byte aligned sources
    nb = 4099 if per == 256 else 4099 * 8
    raw = np.random.default_rng(code * 10 + off).integers(0, 256, nb * size, dtype=np.uint8)
    got = gpu.dequant_gguf_py(_at_offset(raw, off, dev), nb * per, code)
    assert_bits_equal(to_np(got), O.dequant_py(raw, code), f"type {code} offset {off}")


@pytest.mark.parametrize("code", [0, 1])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 4097, 65539])
def test_f16_f32_tails(dev, code, n):
    per, size = gpu.GGUF_PY_BLOCKS[code]
    raw = np.random.default_rng(n + code).integers(0, 256, n * size, dtype=np.uint8)
    got = gpu.dequant_gguf_py(_at_offset(raw, 3, dev), n, code)
    assert_bits_equal(to_np(got), O.dequant_py(raw, code), f"type {code} n {n}")


def test_all_f16_codes(dev):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = gpu.dequant_gguf_py(_d(h.view(np.uint8), dev), h.size, 1)
    assert_bits_equal(to_np(got), h.view(np.float16).astype(np.float32), "every f16 code")
