"""The padded Q8 layout on the GPU (inference/llamatov_c_inference.py:88-100):
conversion bit for bit against the oracle, and the tile-order product on it
bit for bit against the Q8_0 dispatcher on the same blocks."""
import numpy as np
import pytest

from bpd_substrate_amd import gpu, synth
from helpers import assert_bits_equal, special_f32_blocks, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _d(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_q8_0_rows(pad, N, K):
    """Repack records (b, n) into N rows of 34-byte Q8_0 blocks (d, q)."""
    rec = pad.reshape(K // 32, N, 64)
    out = np.empty((N, K // 32, 34), np.uint8)
    out[:, :, 0:2] = rec[:, :, 0:2].transpose(1, 0, 2)
    out[:, :, 2:34] = rec[:, :, 4:36].transpose(1, 0, 2)
    return out.reshape(-1)


@pytest.mark.parametrize("N,K", [(1, 32), (7, 96), (300, 4096), (4096, 14336)])
def test_pad64_conversion(dev, N, K):
    x = (synth.normal_f32(N * K, synth.key(80, N)) * np.float32(0.7)).reshape(N, K)
    x[0, :32] = 0.0
    got = to_np(gpu.q8_pad64(_d(x.ravel(), dev), N, K))
    want = O.q8_pad64(x, N, K)
    assert np.array_equal(got, want), f"pad64 N={N} K={K}: {np.count_nonzero(got != want)} bytes differ"


def test_pad64_non_finite_blocks(dev):
    # NaN blocks (d = 0x7E00, every quant 0), Inf blocks (Inf/Inf quant 0), as numpy
    x = special_f32_blocks(32).reshape(3, 96)
    got = to_np(gpu.q8_pad64(_d(x.ravel(), dev), 3, 96))
    want = O.q8_pad64(x, 3, 96)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} bytes differ"


@pytest.mark.parametrize("mw,mt,K", [(4096, 1, 14336), (14336, 1, 4096), (13, 3, 160), (8, 1, 32), (9, 2, 64)])
def test_pad64_product_equals_q8_0_dispatch(dev, mw, mt, K):
    x = synth.normal_f32(mw * K, synth.key(81, mw)).reshape(mw, K)
    pad = gpu.q8_pad64(_d(x.ravel(), dev), mw, K)
    xq = gpu.quant_q8_0(_d(synth.normal_f32(mt * K, synth.key(82, mt)), dev))
    got = to_np(gpu.qmatmul_q8_pad64(pad, xq, mw, mt, K))
    rows = to_q8_0_rows(to_np(pad), mw, K)
    ref_gpu = to_np(gpu.qmatmul_q8_0_dispatch(_d(rows, dev), xq, mw, mt, K))
    assert np.array_equal(got.view(np.uint32), ref_gpu.view(np.uint32))
    if mw * K <= 4096 * 4096:
        assert_bits_equal(got, O.dispatch_q8_0(rows, to_np(xq), mw, mt, K, "T", nthreads=8), f"pad64 {mw}x{K}")
