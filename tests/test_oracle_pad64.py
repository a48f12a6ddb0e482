"""Pins of the padded Q8 layout restatement (oracle bpdq_o_q8_pad64,
inference/llamatov_c_inference.py:88-100), CPU only:

* numpy's own float32 evaluation of the reference's operations (NEP 50 keeps
  `float32_array / 127.0` in float32; np.round is half-to-even) agrees bit for
  bit on random matrices: a C restatement that computed in double, truncated,
  or rounded half away from zero fails it;
* ties x/d = k + 1/2 with d = 1 go to the even neighbour;
* an all-zero block takes d = 1e-10/127, whose binary16 rounds to +0, and
  quantizes to 0;
* layout probes: one non-zero value per (row, block) lands in record (b, n)
  at byte 4 + j, the scale at bytes 0-1, everything else zero;
* non-finite inputs as numpy computes them: a NaN in a block carries into d
  (float16 0x7E00 for the default NaN) and every quant is 0; an Inf makes
  d = Inf and Inf/Inf a NaN quant, cast to 0.
"""
import warnings

import numpy as np

from helpers import special_f32_blocks
from oracle import oracle as O


def numpy_ops(arr):
    # the reference's own operations, step by step, in numpy
    N, K = arr.shape
    nb = K // 32
    blocks = arr.reshape(N, nb, 32)
    amax = np.max(np.abs(blocks), axis=2, keepdims=True).clip(1e-10)
    d = amax / 127.0
    quants = np.clip(np.round(blocks / d), -128, 127).astype(np.int8)
    q8 = np.zeros((N, nb, 64), dtype=np.uint8)
    q8[:, :, :2] = d.squeeze(-1).astype(np.float16).view(np.uint8).reshape(N, nb, 2)
    q8[:, :, 4:36] = quants.view(np.uint8)
    return q8.transpose(1, 0, 2).copy().flatten()


def test_matches_numpy_float32_semantics():
    rng = np.random.default_rng(12)
    for N, K, scale in [(7, 64, 1.0), (33, 256, 1e-3), (5, 4096, 30.0), (64, 128, 1e-6)]:
        x = (rng.normal(0, 1, (N, K)) * scale).astype(np.float32)
        x[0, :32] = 0.0
        assert np.array_equal(O.q8_pad64(x, N, K), numpy_ops(x)), (N, K)


def test_ties_round_to_even():
    x = np.zeros((1, 32), np.float32)
    x[0, :7] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 126.5]     # amax = 127 -> d = 1 exactly
    out = O.q8_pad64(x, 1, 32)
    q = out[4:36].view(np.int8)
    assert list(q[:7]) == [127, 2, -2, 4, 0, 0, 126]
    assert out[0:2].view(np.float16)[0] == 1.0


def test_zero_block_and_layout_probes():
    N, K = 3, 96
    x = np.zeros((N, K), np.float32)
    out = O.q8_pad64(x, N, K)
    assert not out.any()                                     # d = 1e-10/127 -> f16 +0, q = 0
    for n in range(N):
        for b in range(K // 32):
            for j in (0, 17, 31):
                x = np.zeros((N, K), np.float32)
                x[n, 32 * b + j] = -3.0
                out = O.q8_pad64(x, N, K).reshape(K // 32, N, 64)
                rec = out[b, n]
                assert rec[4 + j].view(np.int8) == -127 and rec[0:2].view(np.float16)[0] == np.float16(3 / 127)
                assert np.count_nonzero(out) == np.count_nonzero(rec) == 3


def test_non_finite_blocks_match_numpy():
    x = special_f32_blocks(32).reshape(3, 96)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # numpy warns on the NaN casts it performs
        want = numpy_ops(x)
    assert np.array_equal(O.q8_pad64(x, 3, 96), want)
    rec = O.q8_pad64(x, 3, 96).reshape(3, 3, 64)   # [block][row]
    for b in (0, 1):  # row 0, blocks 0 (one NaN) and 1 (all NaN): d = 0x7E00, every quant 0
        assert rec[b, 0, 0:2].view(np.uint16)[0] == 0x7E00 and not rec[b, 0, 4:36].any()
    assert rec[2, 0, 0:2].view(np.uint16)[0] == 0x7C00   # row 0, block 2 (an Inf): d = Inf
