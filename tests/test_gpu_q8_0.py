"""GPU parity of the Q8_0 kernels against the C oracle, through the C ABI.

dequant, embed lookup and the quantizer are bit-exact with bench/bpd_cpu.c; the
dispatcher and the llamafile path are bit-exact with the AVX1 build's tile
order T (bench/bpd_gemm_q8_0_cpu.c:32-86).  Int8 values stay in [-127, 127],
the range every Q8_0 quantizer produces.
"""
import numpy as np
import pytest

from bpd_substrate_amd import gpu, synth
from helpers import assert_bits_equal, special_f32_blocks, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _d(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("n_blocks", [1, 3, 128 * 448])
def test_dequant_q8_0(dev, n_blocks):
    raw = synth.q8_0(n_blocks, 32, synth.key(42, 4))
    assert_bits_equal(to_np(gpu.dequant_q8_0(_d(raw, dev))), O.dequant_q8_0(raw), "dequant_q8_0")


def test_dequant_q8_0_subnormal_scale(dev):
    # tests/check_dequant_subnormal.py:9-31: f16 0x00c2 times int8 1 = 194 * 2^-24
    blk = np.array([0xC2, 0x00] + [1] * 32, np.uint8)
    got = to_np(gpu.dequant_q8_0(_d(blk, dev)))
    assert np.all(got == np.float32(194 * 2.0 ** -24))


def test_embed_lookup_q8_0(dev):
    table = synth.q8_0(100, 4096, synth.key(42, 5))
    ids = np.array([3, 0, 99, 3, 57], np.int32)
    got = to_np(gpu.embed_lookup_q8_0(_d(table, dev), _d(ids, dev), 4096))
    assert_bits_equal(got, O.embed_lookup_q8_0(table, ids, 4096), "embed lookup")


@pytest.mark.parametrize("n", [32, 4096, 14336, 512 * 4096])
def test_quant_q8_0(dev, n):
    x = synth.normal_f32(n, synth.key(42, 6))
    got = to_np(gpu.quant_q8_0(_d(x, dev)))
    want = O.quant_q8_0(x)
    assert np.array_equal(got, want), f"Q8_0 bytes differ at {np.flatnonzero(got != want)[:8]}"


def test_quant_q8_0_non_finite(dev):
    # the x86 cast of the reference (0 for NaN and for +-Inf), which the GPU's
    # saturating v_cvt_i32_f32 does not give for +Inf by itself
    x = special_f32_blocks(32)
    got = to_np(gpu.quant_q8_0(_d(x, dev)))
    want = O.quant_q8_0(x)
    assert np.array_equal(got, want), f"bytes differ at {np.flatnonzero(got != want)[:8]}"


def test_quant_q8_0_edges(dev):
    x = np.zeros(6 * 32, np.float32)
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5          # ties at x*id = k + 0.5
    x[64:96] = 6.0e-5 * (np.arange(32) - 16)                    # d in the f16 subnormal range
    x[96:128] = 1.0e5                                           # d = 787.4 -> f16 rounding
    x[128:160] = 9.0e6                                          # amax/127 > 65504: d -> f16 Inf
    x[160] = -0.0
    got = to_np(gpu.quant_q8_0(_d(x, dev)))
    want = O.quant_q8_0(x)
    assert np.array_equal(got, want), f"bytes differ at {np.flatnonzero(got != want)[:8]}"


@pytest.mark.parametrize("mw,mt,K", [(14336, 1, 4096), (4096, 1, 14336), (4, 2, 128), (7, 5, 128),
                                     (9, 7, 128), (2048, 2, 2048), (1, 1, 32), (13, 3, 4096 + 32),
                                     # the wide-load kernel: both load forms, partial last
                                     # workgroups and waves, each activation register count,
                                     # several tokens, an odd chunk count, and 8 waves where 4
                                     # cannot hold the x row (K = 65536, over 64 KB of LDS)
                                     (8192, 2, 1024), (8200, 3, 8192), (2048, 1, 8192), (9000, 1, 2048),
                                     (2056, 1, 16384), (4096, 4, 4096), (4100, 1, 4096), (4096, 1, 4096),
                                     (2048, 1, 32768), (4096, 2, 14336), (511, 1, 4096), (1024, 1, 14336),
                                     (2048, 1, 4096), (514, 1, 1024), (512, 1, 65536), (513, 1, 3072),
                                     (4097, 3, 1024)])
def test_dispatch_tile_order(dev, mw, mt, K):
    W = synth.q8_0(mw, K, synth.key(42, 7))
    X = synth.normal_f32(mt * K, synth.key(42, 8))
    Xq = O.quant_q8_0(X)
    got = to_np(gpu.qmatmul_q8_0_dispatch(_d(W, dev), _d(Xq, dev), mw, mt, K))
    assert_bits_equal(got, O.dispatch_q8_0(W, Xq, mw, mt, K, "T"), f"dispatch {mw}x{mt}x{K}")


@pytest.mark.parametrize("mw,mt,K", [(14336, 1, 4096), (64, 4, 256), (6, 3, 96)])
def test_llamafile_path(dev, mw, mt, K):
    W = synth.q8_0(mw, K, synth.key(42, 9))
    X = synth.normal_f32(mt * K, synth.key(42, 10))
    got = to_np(gpu.qmatmul_q8_0_llamafile(_d(W, dev), _d(X, dev), mw, mt, K))
    assert_bits_equal(got, O.qmatmul_q8_0_llamafile(W, X, mw, mt, K, "T"), "llamafile")


# ------------------------------------------------- prefill GEMM, scalar order S (int8 MFMA)

@pytest.mark.parametrize("mw,mt,K", [(4, 2, 128), (7, 5, 128), (130, 129, 4096 + 32), (1, 1, 32), (256, 256, 64),
                                     (300, 17, 224), (2048, 64, 2048),
                                     # the 64-row form (one workgroup of 8 waves per CU), the last
                                     # with a ragged row panel
                                     (8192, 256, 512), (8192, 256, 384), (4100, 512, 768)])
def test_dispatch_scalar_order(dev, mw, mt, K):
    W = synth.q8_0(mw, K, synth.key(43, 7))
    X = synth.normal_f32(mt * K, synth.key(43, 8))
    Xq = O.quant_q8_0(X)
    got = to_np(gpu.qmatmul_q8_0_dispatch_s(_d(W, dev), _d(Xq, dev), mw, mt, K))
    assert_bits_equal(got, O.dispatch_q8_0(W, Xq, mw, mt, K, "S", nthreads=8), f"S-order {mw}x{mt}x{K}")


@pytest.mark.parametrize("wo,xo", [(2, 1), (1, 3)])
def test_dispatch_scalar_order_unaligned_operands(dev, wo, xo):
    """W and X at byte offsets that are not multiples of 4 (tensor data in a file need
    not be aligned): the launcher takes the kernel without dword staging, and the
    result is the same."""
    import torch

    mw, mt, K = 130, 129, 256
    W = synth.q8_0(mw, K, synth.key(43, 13))
    Xq = O.quant_q8_0(synth.normal_f32(mt * K, synth.key(43, 14)))
    wb = torch.zeros(W.size + 8, dtype=torch.uint8, device=dev)
    xb = torch.zeros(Xq.size + 8, dtype=torch.uint8, device=dev)
    wb[wo:wo + W.size] = _d(W, dev)
    xb[xo:xo + Xq.size] = _d(Xq, dev)
    got = to_np(gpu.qmatmul_q8_0_dispatch_s(wb[wo:wo + W.size], xb[xo:xo + Xq.size], mw, mt, K))
    assert_bits_equal(got, O.dispatch_q8_0(W, Xq, mw, mt, K, "S", nthreads=8), f"S-order offsets {wo},{xo}")


@pytest.mark.parametrize("mw,mt,K", [(130, 129, 512), (7, 7, 96), (256, 130, 4096), (23, 5, 224), (4100, 512, 256)])
def test_dispatch_scalar_order_dense_special_scales(dev, mw, mt, K):
    """Order S (the prefill GEMM's int8-MFMA kernels and the plain one) on dense NaN / Inf
    scales with zero 4-element groups: every cell, NaN bits included, equals the oracle,
    which equals the scalar reference build on such inputs."""
    nb = K // 32
    W, X = _q8_nan_heavy(mw, nb, synth.key(61, mw)), _q8_nan_heavy(mt, nb, synth.key(62, mt))
    got = to_np(gpu.qmatmul_q8_0_dispatch_s(_d(W, dev), _d(X, dev), mw, mt, K))
    want = O.dispatch_q8_0(W, X, mw, mt, K, "S", nthreads=8)
    assert np.isnan(want).any()
    assert_bits_equal(got, want, f"S-order dense special scales {mw}x{mt}x{K}")


@pytest.mark.parametrize("mw,mt,K", [(130, 129, 512), (40, 9, 224)])
def test_dispatch_scalar_order_special_scales(dev, mw, mt, K):
    """Zero, subnormal, infinite and NaN block scales in W and X: the scale products
    come from an MFMA, and each must equal the fp32 product RN(Ad*Bd) (NaNs compared
    as NaN)."""
    nb = K // 32
    W = synth.q8_0(mw, K, synth.key(43, 11)).reshape(mw, nb, 34).copy()
    X = synth.normal_f32(mt * K, synth.key(43, 12))
    Xq = O.quant_q8_0(X).reshape(mt, nb, 34).copy()
    special = [0x0000, 0x8000, 0x0001, 0x83FF, 0x7C00, 0xFC00, 0x7E00, 0x7BFF]
    for i, h in enumerate(special):
        W[(7 * i) % mw, (3 * i) % nb, 0:2] = np.array([h & 0xFF, h >> 8], np.uint8)
        Xq[(5 * i + 1) % mt, (2 * i + 1) % nb, 0:2] = np.array([h & 0xFF, h >> 8], np.uint8)
    W, Xq = W.ravel(), Xq.ravel()
    got = to_np(gpu.qmatmul_q8_0_dispatch_s(_d(W, dev), _d(Xq, dev), mw, mt, K))
    want = O.dispatch_q8_0(W, Xq, mw, mt, K, "S", nthreads=8)
    assert np.isnan(want).any() and np.isinf(want).any()
    assert_bits_equal(got, want, f"S-order special scales {mw}x{mt}x{K}")   # NaN bits included


SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x83FF, 0x7C00, 0xFC00, 0x7E00, 0xFE00, 0x7C01, 0xFD55, 0x7BFF]


def _special(rows, nb, key):
    raw = synth.q8_0(rows, nb * 32, key).reshape(rows, nb, 34).copy()
    for i, h in enumerate(SPECIAL_F16 * 2):
        raw[(7 * i + 3) % rows, (5 * i + 1) % nb, 0:2] = (h & 0xFF, h >> 8)
    return raw.reshape(-1).copy()


# each kernel of the tile-order dispatcher: the producer/consumer kernel (few waves), the
# wide-load kernel (nb % 32 == 0, >= 256 two-row waves; 4 and 16 activation registers),
# the pipelined kernel (>= 1024 eight-row waves) and the plain one (rows too long for LDS)
@pytest.mark.parametrize("mw,mt,K", [(23, 19, 32), (40, 9, 224), (600, 1, 1024), (520, 3, 4096),
                                     (600, 1, 14336), (8192, 1, 4096 + 32), (9, 2, 59392)])
@pytest.mark.parametrize("dense", [False, True])
def test_dispatch_tile_order_nan_bits(dev, mw, mt, K, dense):
    """Zero, subnormal, infinite and NaN scales (with and without payload) in both
    operands, tile order T: every cell, NaN bits included, equals the oracle, which is
    checked against the AVX1 reference build's nine tile kernels on such inputs (each
    tile puts different operands first).  dense: NaN / Inf scales in 40 % of the blocks
    and zero 4-element groups (Inf * 0), several events per lane chain."""
    nb = K // 32
    if dense:
        W, X = _q8_nan_heavy(mw, nb, synth.key(49, mw)), _q8_nan_heavy(mt, nb, synth.key(50, mt))
    else:
        W, X = _special(mw, nb, synth.key(47, mw)), _special(mt, nb, synth.key(48, mt))
    got = to_np(gpu.qmatmul_q8_0_dispatch(_d(W, dev), _d(X, dev), mw, mt, K))
    want = O.dispatch_q8_0(W, X, mw, mt, K, "T", nthreads=8)
    assert np.isnan(want).any()
    assert_bits_equal(got, want, f"tile order NaN bits {mw}x{mt}x{K}")


@pytest.mark.parametrize("mw,mt,K", [(23, 19, 224), (600, 1, 1024), (520, 3, 4096), (600, 1, 14336),
                                     (8192, 1, 4096 + 32), (9, 2, 59392), (7, 7, 96)])
def test_dispatch_tile_order_full_int8_range(dev, mw, mt, K):
    """Random quant bytes over the whole int8 range in both operands: -128 activations
    against negative weights, where SSSE3's sign/maddubs wrap, make the AVX1 build's
    partials differ from the exact dot; every kernel of the dispatcher gives the
    reference's bits (the activation row's -128 sends its cells to the reference-order
    recomputation)."""
    nb = K // 32
    W, X = _q8_full_range(mw, nb, synth.key(59, mw)), _q8_full_range(mt, nb, synth.key(60, mt))
    got = to_np(gpu.qmatmul_q8_0_dispatch(_d(W, dev), _d(X, dev), mw, mt, K))
    assert_bits_equal(got, O.dispatch_q8_0(W, X, mw, mt, K, "T", nthreads=8), f"tile order int8 range {mw}x{mt}x{K}")


@pytest.mark.parametrize("mw,mt,K", [(7, 7, 96), (5, 6, 128), (11, 3, 64), (9, 1, 160), (1, 9, 192), (2, 2, 256)])
def test_dispatch_tile_order_nan_bits_every_tile(dev, mw, mt, K):
    """Row and token counts whose remainders give every reference tile (4, 2 and 1 rows
    by 4, 2 and 1 tokens), dense NaN / Inf scales."""
    nb = K // 32
    for seed in range(3):
        W, X = _q8_nan_heavy(mw, nb, synth.key(51 + seed, mw)), _q8_nan_heavy(mt, nb, synth.key(54 + seed, mt))
        got = to_np(gpu.qmatmul_q8_0_dispatch(_d(W, dev), _d(X, dev), mw, mt, K))
        assert_bits_equal(got, O.dispatch_q8_0(W, X, mw, mt, K, "T"), f"every tile {mw}x{mt}x{K} seed {seed}")


def _q8_nan_heavy(rows, nb, key):
    """Q8_0 rows with 30 % of the 4-element quant groups zero and a special scale
    (zero, subnormal, +-Inf, NaN with and without payload) in 40 % of the blocks."""
    raw = synth.q8_0(rows, nb * 32, key).reshape(rows * nb, 34).copy()
    rng = np.random.default_rng(key)
    groups = raw[:, 2:].reshape(rows * nb, 8, 4)
    groups[rng.random((rows * nb, 8)) < 0.3] = 0
    raw[:, 2:] = groups.reshape(rows * nb, 32)
    pick = rng.random(rows * nb) < 0.4
    h = np.array(SPECIAL_F16, np.uint16)[rng.integers(0, len(SPECIAL_F16), rows * nb)]
    raw[pick, 0] = (h[pick] & 0xFF).astype(np.uint8)
    raw[pick, 1] = (h[pick] >> 8).astype(np.uint8)
    return raw.reshape(-1).copy()


@pytest.mark.parametrize("mw,mt,K", [(23, 19, 32), (130, 131, 512), (40, 9, 224)])
def test_scalar_order_nan_bits_both_forms(dev, mw, mt, K):
    """NaN / Inf scales with and without payload in both operands, so that the first NaN
    of a cell can come from either factor: dispatch_s takes the scalar tiles' bits,
    llamafile_s (through fp32 activations with infinities and NaNs) bpd_qdot's."""
    nb = K // 32
    W, Xq = _special(mw, nb, synth.key(46, mw)), _special(mt, nb, synth.key(47, mt))
    got = to_np(gpu.qmatmul_q8_0_dispatch_s(_d(W, dev), _d(Xq, dev), mw, mt, K))
    want = O.dispatch_q8_0(W, Xq, mw, mt, K, "S", nthreads=8)
    assert np.isnan(want).any()
    assert_bits_equal(got, want, f"dispatch_s NaN bits {mw}x{mt}x{K}")
    X = synth.normal_f32(mt * K, synth.key(48, mt))
    X[::97] = np.inf
    X[5::101] = -np.inf
    X[7::89] = np.nan
    got = to_np(gpu.qmatmul_q8_0_llamafile_s(_d(W, dev), _d(X, dev), mw, mt, K))
    want = O.qmatmul_q8_0_llamafile(W, X, mw, mt, K, "S")
    assert np.isnan(want).any()
    assert_bits_equal(got, want, f"llamafile_s NaN bits {mw}x{mt}x{K}")


def test_dequant_and_embed_q8_0_nan_bits(dev):
    import torch

    raw = synth.random_bytes(4096 * 34, synth.key(49, 1))
    got = to_np(gpu.dequant_q8_0(_d(raw, dev)))
    want = O.dequant_q8_0(raw)
    assert np.isnan(want).any()
    assert_bits_equal(got, want, "Q8_0 dequant of random bytes")
    ids = np.arange(0, 64, 3, dtype=np.int32)
    got = to_np(gpu.embed_lookup_q8_0(_d(raw, dev), torch.from_numpy(ids).to(dev), 2048))
    assert_bits_equal(got, O.embed_lookup_q8_0(raw, ids, 2048), "Q8_0 embed of random bytes")


def test_llamafile_scalar_build_path(dev):
    mw, mt, K = 96, 40, 512
    W = synth.q8_0(mw, K, synth.key(43, 9))
    X = synth.normal_f32(mt * K, synth.key(43, 10))
    got = to_np(gpu.qmatmul_q8_0_llamafile_s(_d(W, dev), _d(X, dev), mw, mt, K))
    assert_bits_equal(got, O.qmatmul_q8_0_llamafile(W, X, mw, mt, K, "S"), "llamafile, scalar build")


def test_prefill_cfg4_full_size_matches_reference_hash(dev):
    # cfg4: W = cfg2 up (14336 x 4096), X = 512 x 4096 N(0,1) -> Q8_0; the expected
    # SHA-256 is that of the reference's scalar-build dispatcher output (tests/golden/make_golden.py)
    import hashlib
    import json
    import os

    hashes = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "hashes.json")))
    W = synth.q8_0(14336, 4096, synth.key(42, synth.STREAM["cfg2_up"]))
    X = synth.normal_f32(512 * 4096, synth.key(42, synth.STREAM["cfg4_x"]))
    Xq = gpu.quant_q8_0(_d(X, dev))
    assert hashlib.sha256(to_np(Xq).tobytes()).hexdigest() == hashes["ref bpd_quant_q8_0_cpu cfg4_x"]
    out = to_np(gpu.qmatmul_q8_0_dispatch_s(_d(W, dev), Xq, 14336, 512, 4096))
    assert hashlib.sha256(out.tobytes()).hexdigest() == hashes["ref scalar dispatch cfg4 512x14336x4096"]


def test_empty_k_gives_zero_cells(dev):
    import torch

    for name in ("bpd_qmatmul_q8_0_dispatch_gpu", "bpd_qmatmul_q8_0_dispatch_s_gpu"):
        out = torch.full((3 * 5,), float("nan"), device=dev)
        gpu.call(name, None, None, out, 5, 3, 0)
        torch.cuda.synchronize()
        assert to_np(out).view(np.uint32).tolist() == [0] * 15, name


def test_dispatch_unaligned_weights_take_the_dword_kernels(dev):
    # W at an address 2 mod 16: the wide-load kernel needs 16-byte rows, so the
    # dispatcher must take k_q8_0_gemv_T, with the same bits
    import torch

    mw, mt, K = 8192, 1, 1024
    W = synth.q8_0(mw, K, synth.key(45, 1))
    Xq = O.quant_q8_0(synth.normal_f32(mt * K, synth.key(45, 2)))
    buf = torch.zeros(W.size + 16, dtype=torch.uint8, device=dev)
    buf[2:2 + W.size].copy_(_d(W, dev))
    out = torch.empty(mw * mt, dtype=torch.float32, device=dev)
    gpu._use_torch_stream()
    gpu.call("bpd_qmatmul_q8_0_dispatch_gpu", buf.data_ptr() + 2, _d(Xq, dev), out, mw, mt, K)
    assert_bits_equal(to_np(out), O.dispatch_q8_0(W, Xq, mw, mt, K, "T"), "unaligned W")


@pytest.mark.parametrize("mw", [7, 15, 17, 23])
def test_dispatch_spare_waves(dev, mw):
    # row counts that leave whole waves of the last workgroup past the end of W
    K = 256
    W = synth.q8_0(mw, K, synth.key(44, mw))
    Xq = O.quant_q8_0(synth.normal_f32(K, synth.key(44, 1)))
    got = to_np(gpu.qmatmul_q8_0_dispatch(_d(W, dev), _d(Xq, dev), mw, 1, K))
    assert_bits_equal(got, O.dispatch_q8_0(W, Xq, mw, 1, K, "T"), f"spare waves mw={mw}")


def test_workspace_growth_inside_capture_is_refused(dev):
    """The llamafile entry quantizes X into its stream's workspace.  Inside graph capture
    it may use the workspace but never grow it (growing drains the stream and
    allocates): a first, larger request during capture fails with BPDQ_ERR_CAPTURE and
    enqueues nothing.  After the same call once outside capture, on the same stream, it
    captures, and the replays give the eager bits."""
    import torch

    mw, mt, K = 64, 3, 8192 + 512          # a size no other test asks for on this new stream
    W = torch.from_numpy(synth.q8_0(mw, K, synth.key(50, 1))).to(dev)
    X = torch.from_numpy(synth.normal_f32(mt * K, synth.key(50, 2))).to(dev)
    s = torch.cuda.Stream()
    out = torch.zeros(mt * mw, device=dev)
    bump = torch.zeros(1, device=dev)
    g = torch.cuda.CUDAGraph()
    code = None
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gpu.lib().bpd_gpu_set_stream(s.cuda_stream)
            try:
                gpu.call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, out, mw, mt, K)
            except gpu.BpdqError as e:
                code = e.code
            bump.add_(1)                    # keeps the captured graph non-empty
    assert code == 6
    eager = to_np(gpu.qmatmul_q8_0_llamafile(W, X, mw, mt, K))
    with torch.cuda.stream(s):
        gpu.lib().bpd_gpu_set_stream(s.cuda_stream)
        gpu.call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, out, mw, mt, K)   # grows, outside capture
        s.synchronize()
        g2 = torch.cuda.CUDAGraph()
        out2 = torch.zeros(mt * mw, device=dev)
        with torch.cuda.graph(g2, stream=s):
            gpu.lib().bpd_gpu_set_stream(s.cuda_stream)
            gpu.call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, out2, mw, mt, K)
    gpu.lib().bpd_gpu_set_stream(None)
    for _ in range(3):
        out2.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert_bits_equal(to_np(out2), eager, "captured llamafile replay")


# ------------------------------------------- bpd_qmatmul_q8_0_cpu's form: orders P and S

def _q8_full_range(rows, nb, key):
    """Q8_0 rows whose quants take every int8 value, -128 included, with realistic scales."""
    raw = synth.random_bytes(rows * nb * 34, key).reshape(rows, nb, 34)
    raw[:, :, :2] = synth.q8_0(rows, nb * 32, key ^ 0x77).reshape(rows, nb, 34)[:, :, :2]
    raw[0, 0, 2:6] = 0x80                               # -128 in both operands for sure
    return raw.reshape(-1).copy()


@pytest.mark.parametrize("M,N,K", [(1, 14336, 4096), (1, 4096, 14336), (3, 37, 224), (2, 9, 32), (5, 17, 4128)])
def test_qdot_grid_orders_P_and_S_full_int8_range(dev, M, N, K):
    nb = K // 32
    Wq, Xq = _q8_full_range(N, nb, synth.key(51, N)), _q8_full_range(M, nb, synth.key(52, M))
    wd, xd = _d(Wq, dev), _d(Xq, dev)
    import torch

    for name, order in (("bpd_qdot_q8_0_q8_0_grid_gpu", "P"), ("bpd_qdot_q8_0_q8_0_grid_s_gpu", "S")):
        out = torch.full((M * N,), float("nan"), device=dev)
        gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
        gpu.call(name, wd, xd, out, M, N, K)
        assert_bits_equal(to_np(out), O.qdot_grid(Wq, Xq, M, N, K, order), f"qdot {order} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(3, 37, 224), (2, 9, 32), (5, 17, 4128), (1, 600, 4096), (4, 64, 96)])
def test_qdot_grid_orders_P_and_S_nan_bits(dev, M, N, K):
    """Dense NaN / Inf scales (with and without payload) and zero quarter sums: orders P
    and S, every cell, NaN bits included, equals the oracle, which is checked against the
    AVX1 and scalar reference builds on such inputs."""
    import torch

    nb = K // 32
    Wq, Xq = _q8_nan_heavy(N, nb, synth.key(57, N)), _q8_nan_heavy(M, nb, synth.key(58, M))
    wd, xd = _d(Wq, dev), _d(Xq, dev)
    for name, order in (("bpd_qdot_q8_0_q8_0_grid_gpu", "P"), ("bpd_qdot_q8_0_q8_0_grid_s_gpu", "S")):
        out = torch.full((M * N,), 1.0, device=dev)
        gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
        gpu.call(name, wd, xd, out, M, N, K)
        want = O.qdot_grid(Wq, Xq, M, N, K, order)
        assert np.isnan(want).any()
        assert_bits_equal(to_np(out), want, f"qdot {order} NaN bits {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 14336, 4096), (4, 300, 4096), (3, 6, 96), (2, 11, 224)])
def test_qmatmul_q8_0_orders_P_and_S(dev, M, N, K):
    import torch

    W = synth.q8_0(N, K, synth.key(53, N))
    X = synth.normal_f32(M * K, synth.key(54, M))
    for name, order in (("bpd_qmatmul_q8_0_gpu", "P"), ("bpd_qmatmul_q8_0_s_gpu", "S")):
        out = torch.full((M * N,), float("nan"), device=dev)
        gpu.lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)
        gpu.call(name, _d(W, dev), _d(X, dev), out, M, N, K)
        assert_bits_equal(to_np(out), O.qmatmul_q8_0(W, X, M, N, K, order), f"qmatmul {order} {M}x{N}x{K}")


@pytest.mark.parametrize("F,mt,K,kind", [(64, 1, 128, "plain"), (128, 5, 512, "plain"), (512, 130, 512, "plain"),
                                         (1024, 256, 4096, "plain"), (256, 129, 256, "special"),
                                         (192, 40, 384, "nan_heavy")])
def test_gemm_swiglu_epilogue(dev, F, mt, K, kind):
    """bpdq_q8_0_gemm_swiglu_s_gpu (the prefill's gate/up with SwiGLU and its Q8_0 rows in
    the order-S GEMM's epilogue, the up tiles handed to the gate rows' waves through LDS):
    every byte equals the oracle's order-S GEMM of each matrix, SwiGLU and Q8_0
    quantization, with special and dense NaN / Inf scales too."""
    import torch
    nb = K // 32
    if kind == "special":
        Wg, Wu, Xq = _special(F, nb, synth.key(71, F)), _special(F, nb, synth.key(72, F)), _special(mt, nb, synth.key(73, mt))
    elif kind == "nan_heavy":
        Wg, Wu, Xq = (_q8_nan_heavy(F, nb, synth.key(74, F)), _q8_nan_heavy(F, nb, synth.key(75, F)),
                      _q8_nan_heavy(mt, nb, synth.key(76, mt)))
    else:
        Wg, Wu = synth.q8_0(F, K, synth.key(77, F)), synth.q8_0(F, K, synth.key(78, F))
        Xq = O.quant_q8_0(synth.normal_f32(mt * K, synth.key(79, mt)))
    g = O.dispatch_q8_0(Wg, Xq, F, mt, K, "S", nthreads=8)
    u = O.dispatch_q8_0(Wu, Xq, F, mt, K, "S", nthreads=8)
    want = O.quant_q8_0(O.swiglu(g, u))
    if kind != "plain":
        assert np.isnan(g).any() or np.isinf(g).any()
    yq = torch.full((mt * F // 32 * 34,), 0xA5, dtype=torch.uint8, device=dev)
    gpu.call("bpdq_q8_0_gemm_swiglu_s_gpu", _d(Wg, dev), _d(Wu, dev), _d(Xq, dev), yq, mt, F, K)
    gpu.check()
    got = to_np(yq)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"
