"""Q6_K on the GPU through the C ABI against the C oracle (both element maps):
dequant bit for bit, Q6_K x Q8_K GEMV bit for bit."""
import numpy as np
import pytest

from bpd_substrate_amd import formats, gpu, synth
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ORDERS = [(formats.ORDER_BPD, 0), (formats.ORDER_GGUF, 1)]


def q6k_blocks(n, seed, realistic=True):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, 210), dtype=np.uint8)
    if realistic:
        b[:, 208:210] = np.abs(rng.normal(0, 0.02, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def _d(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("order,o", ORDERS)
@pytest.mark.parametrize("nb", [1, 3, 4, 5, 4096])
def test_dequant_q6k(dev, order, o, nb):
    b = q6k_blocks(nb, 100 + nb)
    got = to_np(gpu.dequant_q6k(_d(b, dev), order))
    assert_bits_equal(got, O.dequant_q6k(b, o), f"q6k dequant order {o} nb={nb}")


@pytest.mark.parametrize("order,o", ORDERS)
def test_dequant_q6k_random_bytes(dev, order, o):
    b = q6k_blocks(2048, 7, realistic=False)       # every d bit pattern class, NaN/Inf included
    got, want = to_np(gpu.dequant_q6k(_d(b, dev), order)), O.dequant_q6k(b, o)
    assert np.isnan(want).any()
    assert_bits_equal(got, want, f"q6k random-byte dequant order {o}")   # NaN bits included


@pytest.mark.parametrize("order,o", ORDERS)
@pytest.mark.parametrize("M,K", [(1, 256), (5, 512), (64, 4096), (4096, 4096), (7, 4096), (14336, 4096), (17, 14336),
                                 (1024, 14336), (3, 2304)])
def test_qmatmul_q6k_q8k(dev, order, o, M, K):
    w = q6k_blocks(M * K // 256, M + K)
    x = synth.normal_f32(K, synth.key(70, K))
    xq = gpu.quant_q8_k(_d(x, dev))
    y = to_np(gpu.qmatmul_q6k_q8k(_d(w, dev), xq, M, K, order))
    assert_bits_equal(y, O.qmatmul_q6k_q8k(w, to_np(xq), M, K, o, nthreads=8), f"q6k gemv order {o} {M}x{K}")


def test_q6k_empty_and_k0(dev):
    import torch

    y = torch.full((3,), 7.0, device=dev)
    gpu.qmatmul_q6k_q8k(_d(np.zeros(2, np.uint8), dev), _d(np.zeros(4, np.uint8), dev), 3, 0, out=y)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(y), np.zeros(3, np.float32))
