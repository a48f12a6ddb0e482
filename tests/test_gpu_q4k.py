"""GPU parity of the Q4_K / Q8_K kernels against the C oracle, through the C ABI.

Bit-exact everywhere: dequant (both element maps), the reference-order fp32
GEMV, the Q8_K quantizer and the Q4_K x Q8_K GEMV (exact integer sums + the
documented fp32 tree, which the oracle shares).
"""
import numpy as np
import pytest

from bpd_substrate_amd import formats, gpu, synth
from helpers import assert_bits_equal, special_f32_blocks, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _dev_u8(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("n_blocks", [1, 7, 33, 65536])
@pytest.mark.parametrize("order", [formats.ORDER_BPD, formats.ORDER_GGUF])
def test_dequant_q4k_synthetic(dev, n_blocks, order):
    q = synth.q4k(n_blocks, 256, synth.key(42, 0))
    got = to_np(gpu.dequant_q4k(_dev_u8(q, dev), order))
    want = O.dequant_q4k(q) if order == formats.ORDER_BPD else O.dequant_q4k_gguf(q)
    assert_bits_equal(got, want, f"dequant order={order} nb={n_blocks}")


@pytest.mark.parametrize("order", [formats.ORDER_BPD, formats.ORDER_GGUF])
def test_dequant_q4k_random_bytes(dev, order):
    # the reference harness's no-model mode feeds uniform random bytes
    # (bench/verify_quant_gpu.py:240-243): signed zeros, subnormal, Inf and NaN scales
    q = synth.random_bytes(4096 * 144, synth.key(7, 0))
    got = to_np(gpu.dequant_q4k(_dev_u8(q, dev), order))
    want = O.dequant_q4k(q) if order == formats.ORDER_BPD else O.dequant_q4k_gguf(q)
    assert np.isnan(want).sum() > 1000
    # NaN bits included: the bpd map follows the reference C on x86, the GGUF map the
    # reference's CUDA kernel (canonical NaN)
    assert_bits_equal(got, want, "random-byte dequant")


def test_reference_aliases(dev):
    import torch

    q = synth.q4k(64, 256, synth.key(42, 3))
    qd = _dev_u8(q, dev)
    want_bpd, want_gguf = O.dequant_q4k(q), O.dequant_q4k_gguf(q)
    for name in ["dequant_v1_256", "dequant_v1_128", "dequant_v1_64", "dequant_v1_32", "dequant_ilp2",
                 "dequant_multi2", "dequant_multi4", "dequant_multi8", "run_llamacpp", "run_bpd"]:
        out = torch.full((64 * 256,), float("nan"), device=dev)
        gpu.call(name, qd, out, 64)
        torch.cuda.synchronize()
        want = want_gguf if name.startswith("run_") else want_bpd
        assert_bits_equal(to_np(out), want, name)


def test_qgpu_memory_helpers(dev):
    L = gpu.lib()
    q = synth.q4k(16, 256, synth.key(42, 4))
    n = q.size
    d_q = gpu.call("qgpu_alloc", n)
    d_o = gpu.call("qgpu_alloc", 16 * 256 * 4)
    assert d_q and d_o
    gpu.call("qgpu_h2d", d_q, q.ctypes.data, n)
    gpu.call("bpd_dequant_q4k_gpu", d_q, d_o, 16)
    gpu.call("qgpu_sync")
    out = np.empty(16 * 256, np.float32)
    gpu.call("qgpu_d2h", out.ctypes.data, d_o, out.nbytes)
    gpu.call("qgpu_free", d_q)
    gpu.call("qgpu_free", d_o)
    assert L.bpd_gpu_last_error() == 0
    assert_bits_equal(out, O.dequant_q4k(q), "qgpu_* round trip")


@pytest.mark.parametrize("M,K", [(16, 256), (16, 4096), (77, 512), (4096, 4096), (70, 14336), (5, 16640),
                                 (16, 262144), (1030, 512)])
def test_qmatmul_q4k_reference_order(dev, M, K):
    import torch

    w = synth.q4k(M, K, synth.key(42, 10 + M))
    x = synth.normal_f32(K, synth.key(42, 11))
    got = to_np(gpu.qmatmul_q4k(_dev_u8(w, dev), torch.from_numpy(x).to(dev), M, K))
    assert_bits_equal(got, O.qmatmul_q4k(w, x, M, K), f"bpd_qmatmul_q4k_gpu {M}x{K}")


@pytest.mark.parametrize("n", [256, 4096, 14336])
def test_quant_q8_k(dev, n):
    import torch

    x = synth.normal_f32(n, synth.key(42, 1))
    got = to_np(gpu.quant_q8_k(torch.from_numpy(x).to(dev)))
    want = O.quant_q8_k(x)
    assert np.array_equal(got, want), f"Q8_K bytes differ at {np.flatnonzero(got != want)[:8]}"


def test_quant_q8_k_edge_values(dev):
    import torch

    x = np.zeros(4 * 256, np.float32)             # block 0: all zero
    x[256:512] = np.linspace(-3, 3, 256)           # block 1: exact ties appear at x*id = k + 0.5
    x[512] = 1e-30                                 # block 2: tiny amax
    x[768:1024] = -7.25                            # block 3: constant negative (every q = -127)
    got = to_np(gpu.quant_q8_k(torch.from_numpy(x).to(dev)))
    assert np.array_equal(got, O.quant_q8_k(x))


def test_quant_q8_k_non_finite(dev):
    import torch

    x = special_f32_blocks(256)
    got = to_np(gpu.quant_q8_k(torch.from_numpy(x).to(dev)))
    want = O.quant_q8_k(x)
    assert np.array_equal(got, want), f"Q8_K bytes differ at {np.flatnonzero(got != want)[:8]}"


@pytest.mark.parametrize("M,K", [(512, 4096), (4096, 14336)])
def test_fused_quantize_tiny_amax_block(dev, M, K):
    # a block whose 127/amax overflows: the fused GEMV's in-kernel Q8_K must give
    # the x86 cast's 0 quants (and bsums) there, as the oracle's quantizer
    import torch

    w = synth.q4k(M, K, synth.key(46, 1))
    x = synth.normal_f32(K, synth.key(46, 2))
    x[256:512] = np.float32(1e-38) * np.sign(np.linspace(-1, 1, 256, dtype=np.float32))
    got = to_np(gpu.qmatmul_q4k_q8k_fused(_dev_u8(w, dev), torch.from_numpy(x).to(dev), M, K))
    want = O.qmatmul_q4k_q8k(w, O.quant_q8_k(x), M, K, formats.ORDER_BPD)
    assert_bits_equal(got, want, "fused, tiny-amax block")


@pytest.mark.parametrize("order", [formats.ORDER_BPD, formats.ORDER_GGUF])
@pytest.mark.parametrize("M,K", [(4096, 4096), (14336, 4096), (4096, 14336), (1024, 4096),
                                 (1, 256), (5, 512), (13, 2304), (9, 2048 + 256), (8193, 4096),
                                 # dispatch boundaries: the span kernel's last one-row-per-wave
                                 # size and its first two-row one (an odd row count), and the
                                 # two-row wide kernel (more than 8192 rows of fewer than 16 blocks)
                                 (2048, 4096), (2049, 4096), (8200, 2048)])
def test_qmatmul_q4k_q8k(dev, order, M, K):
    import torch

    w = synth.q4k(M, K, synth.key(42, 2))
    x = synth.normal_f32(K, synth.key(42, 3))
    xq = O.quant_q8_k(x)
    got = to_np(gpu.qmatmul_q4k_q8k(_dev_u8(w, dev), _dev_u8(xq, dev), M, K, order))
    want = O.qmatmul_q4k_q8k(w, xq, M, K, order)
    assert_bits_equal(got, want, f"q4k x q8k order={order} {M}x{K}")
    # the GPU quantizer feeding the GEMV gives the same bytes as the oracle's
    xq_gpu = gpu.quant_q8_k(torch.from_numpy(x).to(dev))
    got2 = to_np(gpu.qmatmul_q4k_q8k(_dev_u8(w, dev), xq_gpu, M, K, order))
    assert_bits_equal(got2, want, "GPU-quantized x")


def test_qmatmul_q4k_q8k_k0_and_empty(dev):
    import torch

    y = torch.full((3,), float("nan"), device=dev)
    gpu.call("bpd_qmatmul_q4k_q8k_gpu", None, None, y, 3, 0)
    torch.cuda.synchronize()
    assert to_np(y).view(np.uint32).tolist() == [0, 0, 0]   # empty sum = +0.0
    gpu.call("bpd_qmatmul_q4k_q8k_gpu", None, None, None, 0, 4096)  # M = 0: nothing to do


def test_invalid_arguments_launch_nothing(dev):
    import torch

    w = _dev_u8(synth.q4k(4, 512, synth.key(1, 1)), dev)
    y = torch.full((4,), 5.0, device=dev)
    cases = [
        ("bpd_qmatmul_q4k_q8k_gpu", (w, w, y, 4, 300), gpu.BpdqError),   # K % 256
        ("bpd_qmatmul_q4k_q8k_gpu", (w, None, y, 4, 512), gpu.BpdqError),  # NULL
        ("bpd_qmatmul_q4k_q8k_gpu", (w.data_ptr() + 4, w, y, 4, 512), gpu.BpdqError),  # misaligned
        ("bpd_dequant_q4k_gpu", (w, y, -1), gpu.BpdqError),
    ]
    for name, args, exc in cases:
        with pytest.raises(exc):
            gpu.call(name, *args)
    torch.cuda.synchronize()
    assert to_np(y).tolist() == [5.0] * 4


@pytest.mark.parametrize("M,K", [(64, 2048), (300, 256)])
def test_qmatmul_q4k_reference_order_nan_bits(dev, M, K):
    """Random-byte weights (Inf / NaN d and dmin) against activations holding quiet and
    signalling NaNs of both signs and infinities: every row bit-identical to the
    reference chain on x86, NaN rows included."""
    import torch

    w = synth.random_bytes(M * K // 256 * 144, synth.key(44, M))
    x = synth.normal_f32(K, synth.key(44, K))
    special = np.array([0x7FC00001, 0xFFC00002, 0x7F800003, 0xFF812345, 0x7F800000, 0xFF800000], np.uint32)
    x[np.arange(special.size) * (K // special.size) + 7] = special.view(np.float32)
    for xv in (synth.normal_f32(K, synth.key(45, K)), x):
        y = gpu.qmatmul_q4k(_dev_u8(w, dev), torch.from_numpy(xv).to(dev), M, K)
        want = O.qmatmul_q4k(w, xv, M, K)
        assert np.isnan(want).any()
        assert_bits_equal(to_np(y), want, f"reference-order GEMV NaN bits {M}x{K}")


@pytest.mark.parametrize("M,N,K", [(3, 5, 256), (64, 64, 4096), (7, 300, 512)])
def test_qmm_q4k_matches_the_reference_chain(dev, M, N, K):
    import torch

    A = synth.q4k(M, K, synth.key(55, M))
    B = synth.normal_f32(K * N, synth.key(56, N))
    C = torch.full((M * N,), float("nan"), device=dev)
    gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
    gpu.call("bpd_qmm_q4k_gpu", _dev_u8(A, dev), torch.from_numpy(B).to(dev), C, M, N, K)
    assert_bits_equal(to_np(C), O.qmm_q4k(A, B, M, N, K), f"bpd_qmm_q4k {M}x{N}x{K}")


def test_qmm_q4k_nan_bits(dev):
    import torch

    M, N, K = 6, 5, 512
    A = synth.random_bytes(M * K // 256 * 144, synth.key(57, 1))
    B = synth.normal_f32(K * N, synth.key(57, 2))
    special = np.array([0x7FC00001, 0xFFC00002, 0x7F800003, 0xFF812345, 0x7F800000, 0xFF800000], np.uint32)
    B[np.arange(special.size) * 401 % B.size] = special.view(np.float32)
    C = torch.full((M * N,), 0.0, device=dev)
    gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
    gpu.call("bpd_qmm_q4k_gpu", _dev_u8(A, dev), torch.from_numpy(B).to(dev), C, M, N, K)
    want = O.qmm_q4k(A, B, M, N, K)
    assert np.isnan(want).any()
    assert_bits_equal(to_np(C), want, "bpd_qmm_q4k NaN bits")
