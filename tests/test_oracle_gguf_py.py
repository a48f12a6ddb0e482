"""The oracle's restatement of the reference Python loader's per-type dequant
(load_tensor_by_type, inference/llamatov_helpers.py:196-222), pinned three ways:

* bit for bit against the reference's own functions on the golden blocks
  (tests/golden/gguf_py.npz, written by tests/golden/make_gguf_py_golden.py).
  Those blocks have NaN, Inf, signalling-NaN, subnormal and -0.0 scales, so the
  element maps and the NaN bits are pinned there;
* the F16 decode over all 65,536 codes against numpy's astype, which is what the
  reference's F16 branch (:205-207) calls;
* each formula on finite blocks against the same value computed exactly in
  binary64 and rounded once. Every product in these formulas is exact in fp32,
  so only the final difference rounds. A dropped term, a wrong nibble or a swapped
  scale fails this check."""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "gguf_py.npz")
TYPES = {"q4_0": 2, "q2_k": 10, "q3_k": 11, "q4_k": 12}


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


@pytest.mark.parametrize("name", list(TYPES))
def test_matches_reference_python(gold, name):
    got = O.dequant_py(gold[name + "_blocks"], TYPES[name])
    want = gold[name + "_dequant"]
    assert np.isnan(want).any() and np.isinf(want).any()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


def test_f16_matches_reference_python_and_numpy(gold):
    got = O.dequant_py(gold["f16_bits"].view(np.uint8), 1)
    assert np.array_equal(got.view(np.uint32), gold["f16_dequant"].view(np.uint32))
    allc = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.dequant_py(allc.view(np.uint8), 1)
    assert np.array_equal(got.view(np.uint32), allc.view(np.float16).astype(np.float32).view(np.uint32))


def test_f32_is_a_copy():
    x = np.random.default_rng(3).integers(0, 2**32, 77, dtype=np.uint32)
    assert np.array_equal(O.dequant_py(x.view(np.uint8), 0).view(np.uint32), x)


def _finite_blocks(size, offs, n, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, size), dtype=np.uint8)
    for o in offs:
        b[:, o:o + 2] = rng.normal(0, 3, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b


def _f16(b, o):
    return b[:, o:o + 2].copy().view(np.float16).astype(np.float64).ravel()


def test_formulas_in_exact_arithmetic():
    n = 40
    # Q4_0: d * (q - 8), element e < 16 low nibble of qs[e], 16 + e high nibble
    b = _finite_blocks(18, (0,), n, 1)
    q = np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4], 1).astype(np.float64)
    want = (_f16(b, 0)[:, None] * (q - 8)).astype(np.float32)
    assert np.array_equal(O.dequant_py(b, 2).reshape(n, 32), want)
    # Q2_K: (scales & 15) * d * q - (scales >> 4) * dmin, q = bits 2(e%4) of qs[e/4]
    b = _finite_blocks(84, (80, 82), n, 2)
    e = np.arange(256)
    q = ((b[:, 16 + e // 4] >> (2 * (e % 4))) & 3).astype(np.float64)
    s = b[:, e // 16].astype(np.int64)
    want = ((s & 15) * _f16(b, 80)[:, None] * q - (s >> 4) * _f16(b, 82)[:, None]).astype(np.float32)
    assert np.array_equal(O.dequant_py(b, 10).reshape(n, 256), want)
    # Q3_K (approximate): d * (nibble(scales[i % 8], i / 8) - 8) * (q + 4 hbit - 4)
    b = _finite_blocks(110, (108,), n, 3)
    i = e // 16
    sb = b[:, 96 + (i % 8)].astype(np.int64)
    scale = np.where(i < 8, sb & 15, sb >> 4) - 8
    quant = ((b[:, 32 + e // 4] >> (2 * (e % 4))) & 3) + 4 * ((b[:, e // 8] >> (e % 8)) & 1) - 4
    want = (_f16(b, 108)[:, None] * scale * quant).astype(np.float32)
    assert np.array_equal(O.dequant_py(b, 11).reshape(n, 256), want)
    # Q4_K: d * sc_j * q - dmin * m_j; e < 128 low nibble of qs[e] (j = e/32), else high of qs[e-128]
    b = _finite_blocks(144, (0, 2), n, 4)
    sc6, m6 = np.zeros((n, 8), np.int64), np.zeros((n, 8), np.int64)
    S = b[:, 4:16].astype(np.int64)
    for j in range(4):
        sc6[:, j], m6[:, j] = S[:, j] & 63, S[:, j + 4] & 63
        sc6[:, j + 4] = (S[:, j + 8] & 15) | ((S[:, j] >> 6) << 4)
        m6[:, j + 4] = (S[:, j + 8] >> 4) | ((S[:, j + 4] >> 6) << 4)
    qs = b[:, 16:144].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], 1)
    j = np.where(e < 128, (e % 128) // 32, 4 + (e % 128) // 32)
    want = (_f16(b, 0)[:, None] * sc6[:, j] * q - _f16(b, 2)[:, None] * m6[:, j]).astype(np.float32)
    assert np.array_equal(O.dequant_py(b, 12).reshape(n, 256), want)


def test_plausible_mistakes_fail():
    """The exact-arithmetic check above tells the formulas apart: swapping Q4_0's
    nibble halves, or Q4_K's map for the GGUF one, changes the output."""
    b = _finite_blocks(18, (0,), 8, 5)
    sw = b.copy()
    sw[:, 2:] = ((b[:, 2:] & 15) << 4) | (b[:, 2:] >> 4)
    assert not np.array_equal(O.dequant_py(b, 2), O.dequant_py(sw, 2))
    b = _finite_blocks(144, (0, 2), 8, 6)
    assert not np.array_equal(O.dequant_py(b, 12), O.dequant_q4k_gguf(b.ravel()))
