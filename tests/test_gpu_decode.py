"""GPU parity of the decode-step GEMV chain (Mistral-7B shapes) and of the fused
multi-matrix GEMV, through the C ABI, against the C oracle."""
import numpy as np
import pytest

from bpd_substrate_amd import decode, gpu, synth
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _d(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_multi_matches_single(dev):
    K = 4096
    shapes = [4096, 1024, 1024, 13]
    ws = [synth.q4k(m, K, synth.key(50, i)) for i, m in enumerate(shapes)]
    xq = gpu.quant_q8_k(_d(synth.normal_f32(K, synth.key(50, 9)), dev))
    wd = [_d(w, dev) for w in ws]
    outs = gpu.qmatmul_q4k_q8k_multi(wd, xq, shapes, K)
    xq_h = to_np(xq)
    for w, o, m in zip(ws, outs, shapes):
        assert_bits_equal(to_np(o), O.qmatmul_q4k_q8k(w, xq_h, m, K, 0), f"multi rows={m}")


def test_multi_long_rows(dev):
    K = 14336
    shapes = [4096, 33]
    ws = [synth.q4k(m, K, synth.key(51, i)) for i, m in enumerate(shapes)]
    xq = gpu.quant_q8_k(_d(synth.normal_f32(K, synth.key(51, 9)), dev))
    outs = gpu.qmatmul_q4k_q8k_multi([_d(w, dev) for w in ws], xq, shapes, K)
    for w, o, m in zip(ws, outs, shapes):
        assert_bits_equal(to_np(o), O.qmatmul_q4k_q8k(w, to_np(xq), m, K, 0), f"multi K=14336 rows={m}")


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 4096), (4096, 14336), (1024, 4096), (6144, 4096), (5, 512),
                                 (3, 256), (17, 8192), (40, 16384), (9, 16640), (7, 0)])
def test_fused_matches_oracle(dev, M, K):
    """fp32 x quantized inside the GEMV (K > 16384 takes the two-launch path)."""
    w = synth.q4k(M, K, synth.key(52, M)) if K else np.zeros(0, np.uint8)
    x = synth.normal_f32(K, synth.key(52, K + 1)) if K else np.zeros(0, np.float32)
    if K:
        x[:256] = 0.0                       # an all-zero block: d = 0, id = 0
        x[256:260] *= 1e4                    # a block dominated by a few large values
    wd = _d(w, dev) if K else _d(np.zeros(16, np.uint8), dev)
    xd = _d(x, dev) if K else _d(np.zeros(4, np.float32), dev)
    y = gpu.qmatmul_q4k_q8k_fused(wd, xd, M, K)
    want = O.qmatmul_q4k_q8k(w, O.quant_q8_k(x), M, K, 0, nthreads=8) if K else np.zeros(M, np.float32)
    assert_bits_equal(to_np(y), want, f"fused M={M} K={K}")


def test_fused_edge_values_match_two_launches(dev):
    """Quantizer edge values (signed zeros, subnormals, near-FLT_MAX, NaN): the fused kernel
    and bpd_quant_q8_k_gpu + bpd_qmatmul_q4k_q8k_gpu give the same bits."""
    import torch

    K, M = 2048, 300
    x = synth.normal_f32(K, synth.key(53, 1))
    x[0:256] = -0.0
    x[256:512] *= 1e-42                     # subnormal block
    x[512:768] = np.float32(3.0e38) * np.sign(x[512:768])
    x[768] = np.nan
    x[1024:1280] = np.nan
    w = _d(synth.q4k(M, K, synth.key(53, 2)), dev)
    xd = _d(x, dev)
    y1 = gpu.qmatmul_q4k_q8k_fused(w, xd, M, K)
    y2 = gpu.qmatmul_q4k_q8k(w, gpu.quant_q8_k(xd), M, K)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(y1).view(np.uint32), to_np(y2).view(np.uint32))


def test_fused_multi_matches_multi(dev):
    K = 4096
    shapes = [4096, 1024, 1024]
    ws = [_d(synth.q4k(m, K, synth.key(54, i)), dev) for i, m in enumerate(shapes)]
    x = _d(synth.normal_f32(K, synth.key(54, 9)), dev)
    a = gpu.qmatmul_q4k_q8k_fused_multi(ws, x, shapes, K)
    b = gpu.qmatmul_q4k_q8k_multi(ws, gpu.quant_q8_k(x), shapes, K)
    for u, v, m in zip(a, b, shapes):
        assert np.array_equal(to_np(u).view(np.uint32), to_np(v).view(np.uint32)), f"rows={m}"


@pytest.mark.parametrize("fused", [True, False])
def test_decode_chain_two_layers(dev, fused):
    d = decode.Dims()
    e, kv, ff = d.n_embd, d.n_kv, d.ff
    host, layers = [], []
    for i in range(2):
        k = lambda t: synth.key(42, 1000 + 8 * i + t)
        h = dict(q=synth.q4k(e, e, k(0)), k=synth.q4k(kv, e, k(1)), v=synth.q4k(kv, e, k(2)), o=synth.q4k(e, e, k(3)),
                 gate=synth.q4k(ff, e, k(4)), up=synth.q4k(ff, e, k(5)), down=synth.q4k(e, ff, k(6)))
        host.append(h)
        layers.append(decode.LayerWeights(**{n: _d(v, dev) for n, v in h.items()}))
    acts_h = [[synth.normal_f32(n, synth.key(43, 10 * i + j)) for j, n in enumerate((e, e, e, ff))] for i in range(2)]
    acts = [[_d(a, dev) for a in la] for la in acts_h]
    chain = decode.GemvChain(layers, d, fused=fused)
    gpu.lib().bpd_gpu_set_stream(None)
    chain.step(acts)
    gpu.check()
    import torch

    torch.cuda.synchronize()
    for i in range(2):
        xa, xo, xf, xh = (O.quant_q8_k(a) for a in acts_h[i])
        want = dict(q=(xa, e, e), k=(xa, kv, e), v=(xa, kv, e), o=(xo, e, e), gate=(xf, ff, e), up=(xf, ff, e),
                    down=(xh, e, ff))
        for name, (xq, M, K) in want.items():
            assert_bits_equal(to_np(chain.out[i][name]), O.qmatmul_q4k_q8k(host[i][name], xq, M, K, 0, nthreads=8),
                              f"layer {i} {name}")
