"""Pin the oracle where the reference has no code, or beyond its fixtures, by
mathematics: exhaustive KATs, closed forms, element-map probes, brute-force
integer sums.  Each check is built so that a plausible slip in the oracle (a
dropped term, a wrong sign, a transposed index, a wrong rounding) fails it.
"""
import ctypes

import numpy as np
import pytest

from bpd_substrate_amd import synth
from helpers import assert_bits_equal
from oracle import oracle as O

L = O.lib


def f16_table():
    h = np.arange(65536, dtype=np.uint16)
    return h, h.view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- f16

def test_f16_decoders_exhaustive_vs_ieee():
    # tests/check_f16_algorithm.py:85-117 runs the same exhaustive comparison against numpy
    h, want = f16_table()
    nan = np.isnan(want)
    for name in ("bpdq_o_f16_ldexp", "bpdq_o_f16_magic", "bpdq_o_f16_h2h"):
        fn = getattr(L(), name)
        got = np.array([fn(int(v)) for v in h], np.float32)
        w = want.copy()
        if name == "bpdq_o_f16_h2h":   # both zeros -> +0, NaN -> Inf (bench_dequant_gpu_h2h.cu:16-17)
            w[h == 0x8000] = 0.0
            w[nan] = np.where(h[nan] & 0x8000, -np.inf, np.inf)
            assert_bits_equal(got, w, name)
            continue
        assert_bits_equal(got[~nan], w[~nan], name)
        assert np.all(np.isnan(got[nan]))
        if name == "bpdq_o_f16_magic":  # payload kept, quiet bit set
            bits = got[nan].view(np.uint32)
            hb = h[nan].astype(np.uint32)
            assert np.array_equal(bits, ((hb & 0x8000) << 16) | 0x7F800000 | ((hb & 0x3FF) << 13) | 0x400000)


def test_f16_subnormal_kat():
    # tests/check_dequant_subnormal.py:9-31: 0x00c2 -> 194 * 2^-24
    for name in ("bpdq_o_f16_ldexp", "bpdq_o_f16_magic", "bpdq_o_f16_h2h"):
        assert getattr(L(), name)(0x00C2) == np.float32(194 * 2.0 ** -24)


def test_f32_to_f16_vs_ieee_rne():
    rng = np.random.default_rng(1)
    bits = np.concatenate([
        rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32),
        np.arange(0x33000000 - 64, 0x33000000 + 64, dtype=np.uint32),      # half of the smallest subnormal
        np.arange(0x38800000 - 64, 0x38800000 + 64, dtype=np.uint32),      # subnormal/normal boundary
        np.arange(0x477FEFC0, 0x477FF040, dtype=np.uint32),                # overflow boundary 65520
        np.array([0, 0x80000000, 0x7F800000, 0xFF800000], np.uint32),
    ])
    f = bits.view(np.float32)
    ok = ~np.isnan(f)
    got = np.array([L().bpdq_o_f32_to_f16(float(v)) for v in f[ok]], np.uint16)
    with np.errstate(over="ignore"):
        want = f[ok].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- Q4_K

def test_q4k_dequant_closed_form():
    # y = d*sc*q - dmin*m: the double-precision expression is exact for these
    # magnitudes, so the single binary32 rounding of it is the only correct answer
    q = synth.q4k(512, 256, synth.key(21, 1))
    blk = q.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    s = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((len(blk), 8), np.int64)
    mn = np.zeros((len(blk), 8), np.int64)
    sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blk[:, 16:].astype(np.int64).reshape(-1, 8, 16)
    nib = np.concatenate([qs & 15, qs >> 4], axis=2)          # bpd map: [j][k<16 low, k>=16 high]
    exact = d[:, None, None] * sc[:, :, None] * nib - dm[:, None, None] * mn[:, :, None]
    assert_bits_equal(O.dequant_q4k(q), exact.astype(np.float32).ravel(), "closed form")


def _scale_min(blk):
    s = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((len(blk), 8), np.int64)
    mn = np.zeros((len(blk), 8), np.int64)
    sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def test_q4k_gguf_dequant_nan_is_the_cuda_canonical_nan():
    # random bytes: the h2h decode turns NaN scales into +/-Inf, so NaNs come only from
    # Inf*0 and Inf-Inf.  Every other value is numpy's float32 d1*q - m1 (exact products,
    # one rounding), every NaN is 0x7FFFFFFF, the NaN the reference's CUDA kernel returns.
    q = synth.random_bytes(2048 * 144, synth.key(21, 2))
    blk = q.reshape(-1, 144)
    h = blk[:, 0:4].copy().view(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    f[(h & 0x7C00) == 0x7C00] = np.where(h[(h & 0x7C00) == 0x7C00] & 0x8000, -np.inf, np.inf)
    f[(h & 0x7FFF) == 0] = 0.0
    sc, mn = _scale_min(blk)
    qs = blk[:, 16:].astype(np.float32).reshape(-1, 4, 32)
    y = np.empty((len(blk), 4, 2, 32), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for i in range(4):
            for hi in range(2):
                j = 2 * i + hi
                nib = np.floor(qs[:, i] / 16) if hi else qs[:, i] % 16
                y[:, i, hi] = (f[:, 0:1] * sc[:, j:j + 1].astype(np.float32)) * nib - \
                    f[:, 1:2] * mn[:, j:j + 1].astype(np.float32)
    y = y.ravel()
    assert np.isnan(y).sum() > 100
    y.view(np.uint32)[np.isnan(y)] = 0x7FFFFFFF
    assert_bits_equal(O.dequant_q4k_gguf(q), y, "GGUF map, random bytes")


@pytest.mark.parametrize("order", [0, 1])
def test_q4k_element_map_probes(order):
    # one non-zero nibble per probe block; d = 1, every scale 1, dmin = 0 -> a single 1.0
    blocks = np.zeros((256, 144), np.uint8)
    blocks[:, 1] = 0x3C                       # d = 1.0
    blocks[:, 4:8] = 1
    blocks[:, 12:16] = 1
    for p in range(256):
        byte, hi = p % 128, p // 128
        blocks[p, 16 + byte] = 0x10 if hi else 0x01
    deq = (O.dequant_q4k if order == 0 else O.dequant_q4k_gguf)(blocks.ravel()).reshape(256, 256)
    for p in range(256):
        byte, hi = p % 128, p // 128
        if order == 0:   # bench/bpd_quant.c:68-72
            e = 32 * (byte // 16) + 16 * hi + byte % 16
        else:            # bench/bench_dequant_gpu_h2h.cu:31-46 (llama.cpp dequantize_row_q4_K)
            e = 64 * (byte // 32) + 32 * hi + byte % 32
        nz = np.flatnonzero(deq[p])
        assert nz.tolist() == [e], (p, nz.tolist(), e)


# ---------------------------------------------------------------- Q8_K

def test_q8k_quantizer_matches_reference_q8_0_rule():
    # With the same amax in every 32-element sub-block, the Q8_K quantizer must
    # produce the Q8_0 quantizer's int8 values (same id = 127/amax, same rint).
    x = synth.normal_f32(16 * 256, synth.key(22, 1)).reshape(16, 8, 32)
    amax = np.abs(x).max(axis=(1, 2))
    x[:, :, 0] = amax[:, None] * np.where(np.arange(8) % 2, -1, 1)[None, :]
    x = x.reshape(-1).astype(np.float32)
    q8k = O.quant_q8_k(x).reshape(16, 292)
    q80 = O.quant_q8_0(x).reshape(16, 8, 34)
    assert np.array_equal(q8k[:, 4:260].view(np.int8).reshape(16, 8, 32), q80[:, :, 2:].view(np.int8))
    d = q8k[:, 0:4].copy().view(np.float32).ravel()
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    bs = q8k[:, 260:292].copy().view(np.int16)
    assert np.array_equal(bs, q8k[:, 4:260].view(np.int8).reshape(16, 16, 16).astype(np.int16).sum(axis=2))


def test_q8k_quantizer_edges():
    x = np.zeros(3 * 256, np.float32)
    x[256:512] = 2.0                     # q = 127 everywhere
    x[600] = -5.0                        # block 2: one non-zero, negative
    y = O.quant_q8_k(x).reshape(3, 292)
    assert y[0].tolist() == [0] * 292
    assert np.all(y[1, 4:260].view(np.int8) == 127) and np.all(y[1, 260:].copy().view(np.int16) == 127 * 16)
    q = y[2, 4:260].view(np.int8)
    assert q[600 - 512] == -127 and np.count_nonzero(q) == 1


# ---------------------------------------------------------------- Q4_K x Q8_K

def _deq_with(blocks, d_bits, dmin_bits, gguf):
    b = blocks.reshape(-1, 144).copy()
    b[:, 0], b[:, 1] = d_bits & 0xFF, d_bits >> 8
    b[:, 2], b[:, 3] = dmin_bits & 0xFF, dmin_bits >> 8
    return (O.dequant_q4k_gguf if gguf else O.dequant_q4k)(b.ravel()).reshape(-1, 256)


@pytest.mark.parametrize("order", [0, 1])
def test_q4k_q8k_integer_sums_brute_force(order):
    # With d = 1, dmin = 0 the dequant gives sc_j*q(e) for every element e (in the
    # element map under test); with d = 0, dmin = 1 it gives -m_j.  So
    # I = sum_e deq1(e) x(e) and Mn = -sum_e deq2(e) x(e), exactly, in int64.
    w = synth.q4k(64, 256, synth.key(23, order))
    x = synth.normal_f32(64 * 256, synth.key(23, 9))
    xq = O.quant_q8_k(x).reshape(64, 292)
    xi = xq[:, 4:260].view(np.int8).astype(np.int64)
    d1 = _deq_with(w, 0x3C00, 0x0000, order).astype(np.int64)
    d2 = _deq_with(w, 0x0000, 0x3C00, order)
    for b in range(64):
        I_, M_ = O.block_ints(w.reshape(64, 144)[b].copy(), xq[b].copy(), order)
        assert I_ == int((d1[b] * xi[b]).sum())
        assert M_ == int(-(d2[b].astype(np.int64) * xi[b]).sum())


def test_q4k_q8k_single_block_exact_value():
    # d = 1, dy = 1 (amax 127): every product is exact, so y = I - Mn exactly.
    w = synth.q4k(1, 256, synth.key(24, 1)).reshape(144)
    w[0:2] = [0x00, 0x3C]
    w[2:4] = [0x00, 0x3C]
    x = synth.normal_f32(256, synth.key(24, 2))
    x = np.round(x * 30).astype(np.float32)
    x[0] = 127.0
    xq = O.quant_q8_k(x)
    assert xq[:4].view(np.float32)[0] == 1.0
    I_, M_ = O.block_ints(w, xq, 0)
    y = O.qmatmul_q4k_q8k(w, xq, 1, 256, 0)
    assert y[0] == np.float32(I_ - M_) and abs(I_ - M_) < 2**24


@pytest.mark.parametrize("M,K", [(64, 4096), (16, 14336)])
def test_q4k_q8k_close_to_exact_dot(M, K):
    # the fp32 result is within a few ulp of sum |terms| of the exact rational value
    w = synth.q4k(M, K, synth.key(25, K))
    x = synth.normal_f32(K, synth.key(25, 1))
    xq = O.quant_q8_k(x)
    y = O.qmatmul_q4k_q8k(w, xq, M, K, 0).astype(np.float64)
    nb = K // 256
    xqb = xq.reshape(nb, 292)
    dy = xqb[:, 0:4].copy().view(np.float32).astype(np.float64).ravel()
    for r in range(M):
        blocks = w.reshape(M, nb, 144)[r]
        exact, mag = 0.0, 0.0
        for b in range(nb):
            I_, M_ = O.block_ints(blocks[b].copy(), xqb[b].copy(), 0)
            d = float(blocks[b, 0:2].copy().view(np.float16)[0])
            dm = float(blocks[b, 2:4].copy().view(np.float16)[0])
            t = d * dy[b] * I_ - dm * dy[b] * M_
            exact += t
            mag += abs(d * dy[b] * I_) + abs(dm * dy[b] * M_)
        assert abs(y[r] - exact) <= 8 * nb * 2.0 ** -24 * mag + 1e-30


# ---------------------------------------------------------------- Q8_0

def test_q8_0_quantizer_kats():
    x = np.zeros(4 * 32, np.float32)
    x[0:32] = np.arange(32, dtype=np.float32) - 15.5    # amax 15.5: x*id hits k+0.5 exactly -> even
    x[32:64] = 0.0                                       # amax 0: d = 0, all q = 0
    x[64:96] = np.where(np.arange(32) % 2, 3.0, -3.0)     # +/-amax -> +/-127
    x[96:128] = 1e-7 * (np.arange(32) - 16)              # d = amax/127 in the f16 subnormal range
    y = O.quant_q8_0(x).reshape(4, 34)
    q = y[:, 2:].view(np.int8)
    xid = x[0:32] * np.float32(127.0 / 15.5)
    assert np.array_equal(q[0], np.rint(xid).astype(np.int8))   # rint = ties to even
    assert y[1].tolist() == [0] * 34
    assert np.array_equal(q[2], np.where(np.arange(32) % 2, 127, -127))
    for b in range(4):
        amax = np.abs(x[32 * b:32 * b + 32]).max()
        assert y[b, 0:2].copy().view(np.float16)[0] == np.float16(np.float32(amax) / np.float32(127))


def test_q8_0_orders_agree_on_exact_inputs():
    # With every scale a power of two and small ints, every fp32 operation is exact,
    # so S, P and T must all give the exact integer dot product.
    nb = 9
    w = synth.q8_0(1, nb * 32, synth.key(26, 1)).reshape(nb, 34)
    a = synth.q8_0(1, nb * 32, synth.key(26, 2)).reshape(nb, 34)
    w[:, 0:2] = [0x00, 0x3C]          # 1.0
    a[:, 0:2] = [0x00, 0x38]          # 0.5
    exact = 0.5 * int((w[:, 2:].view(np.int8).astype(np.int64) * a[:, 2:].view(np.int8)).sum())
    wp, ap = w.ravel().copy(), a.ravel().copy()
    for fn in ("bpdq_o_qdot_q8_0_S", "bpdq_o_qdot_q8_0_P", "bpdq_o_cell_q8_0_T"):
        assert getattr(L(), fn)(wp.ctypes.data, ap.ctypes.data, nb) == exact, fn


def test_q8_0_tile_order_is_not_the_scalar_order():
    # guard against the oracle collapsing T onto S: on random data they differ somewhere
    W = synth.q8_0(256, 4096, synth.key(27, 1))
    X = O.quant_q8_0(synth.normal_f32(4096, synth.key(27, 2)))
    t = O.dispatch_q8_0(W, X, 256, 1, 4096, "T")
    s = O.dispatch_q8_0(W, X, 256, 1, 4096, "S")
    assert np.any(t.view(np.uint32) != s.view(np.uint32))
    assert np.allclose(t, s, rtol=1e-4, atol=1e-4)


def test_multithreaded_wrappers_keep_bits():
    w = synth.q4k(333, 1024, synth.key(28, 1))
    xq = O.quant_q8_k(synth.normal_f32(1024, synth.key(28, 2)))
    assert_bits_equal(O.qmatmul_q4k_q8k(w, xq, 333, 1024, 0, nthreads=7), O.qmatmul_q4k_q8k(w, xq, 333, 1024, 0), "mt")
    assert_bits_equal(O.dequant_q4k_mt(w, 5), O.dequant_q4k(w), "dequant mt")
    W = synth.q8_0(77, 256, synth.key(28, 3))
    X = O.quant_q8_0(synth.normal_f32(3 * 256, synth.key(28, 4)))
    assert_bits_equal(O.dispatch_q8_0(W, X, 77, 3, 256, "T", nthreads=6), O.dispatch_q8_0(W, X, 77, 3, 256, "T"), "mt")
    _ = ctypes  # noqa
