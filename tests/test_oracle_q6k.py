"""Pins of the Q6_K restatement in oracle/bpdq_oracle.c (CPU only).

* order 0 (inference/llamatov_helpers.py:161-179): bit-exact against golden
  vectors the reference's own Python function produced
  (tests/golden/make_q6k_golden.py);
* order 1 (GGUF, llama.cpp dequantize_row_q6_K): element-map probes, one
  non-zero nibble or bit pair at a time, against the published layout, and
  a bijection check;
* both: dequant = d*sc*q rounded once (fp64 closed form); the Q6_K x Q8_K
  integer sums against int64 brute force from the dequant with d = 1; the fp32
  combine on single blocks; full rows within an error bound of the exact sum.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


def block(d=0x3C00, sc=1, ql=0, qh=0):
    b = np.zeros(210, np.uint8)
    b[:128] = ql
    b[128:192] = qh
    b[192:208] = np.int8(sc).view(np.uint8) if np.isscalar(sc) else np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([d & 0xFF, d >> 8], np.uint8)
    return b


def test_order0_matches_reference_python():
    z = np.load(os.path.join(HERE, "golden", "q6k.npz"))
    got = O.dequant_q6k(z["blocks"], 0)
    assert np.array_equal(got.view(np.uint32), z["dequant_ref_order"].view(np.uint32))


def _gguf_element(ql_byte=None, nib=None, qh_byte=None, pair=None):
    """Element a single ql nibble or qh bit pair feeds in llama.cpp's Q6_K layout."""
    if ql_byte is not None:
        # ql[l] feeds y[l] (low) and y[l+64] (high); ql[l+32] feeds y[l+32] and y[l+96]
        h, r = divmod(ql_byte, 64)
        return 128 * h + r + 64 * nib
    h, l = divmod(qh_byte, 32)
    return 128 * h + 32 * pair + l


@pytest.mark.parametrize("order", [0, 1])
def test_element_map_probes(order):
    base = O.q6k_quants(block(), order)
    assert (base == -32).all()
    seen_ql, seen_qh = set(), set()
    for byte in range(128):
        for nib in (0, 1):
            b = block(ql=0)
            b[byte] = 1 << (4 * nib)               # that nibble = 1: q goes -32 -> -31
            q = O.q6k_quants(b, order)
            (e,) = np.flatnonzero(q != -32)
            assert q[e] == -31
            want = (2 * byte + nib) if order == 0 else _gguf_element(ql_byte=byte, nib=nib)
            assert e == want, (byte, nib, e, want)
            seen_ql.add(e)
    for byte in range(64):
        for pair in range(4):
            b = block()
            b[128 + byte] = 1 << (2 * pair)        # high part = 1: q goes -32 -> -16
            q = O.q6k_quants(b, order)
            (e,) = np.flatnonzero(q != -32)
            assert q[e] == -16
            want = (4 * byte + pair) if order == 0 else _gguf_element(qh_byte=byte, pair=pair)
            assert e == want, (byte, pair, e, want)
            seen_qh.add(e)
    assert seen_ql == seen_qh == set(range(256))


def test_gguf_probe_table_is_the_published_layout():
    # spot values of dequantize_row_q6_K: y[l], y[l+32], y[l+64], y[l+96] of each half
    assert _gguf_element(ql_byte=5, nib=0) == 5 and _gguf_element(ql_byte=5, nib=1) == 69
    assert _gguf_element(ql_byte=37, nib=0) == 37 and _gguf_element(ql_byte=37, nib=1) == 101
    assert _gguf_element(ql_byte=64 + 3, nib=1) == 128 + 67
    assert [_gguf_element(qh_byte=32 + 7, pair=p) for p in range(4)] == [135, 167, 199, 231]


@pytest.mark.parametrize("order", [0, 1])
def test_dequant_closed_form(order):
    rng = np.random.default_rng(3)
    b = rng.integers(0, 256, (200, 210), dtype=np.uint8)
    b[:, 208:210] = np.abs(rng.normal(0, 0.05, 200)).astype(np.float16).view(np.uint8).reshape(200, 2)
    b[0, 208:210] = [0x01, 0x00]                   # subnormal d
    b[1, 208:210] = [0xFF, 0x7B]                   # 65504
    got = O.dequant_q6k(b.reshape(-1), order).reshape(200, 256)
    for i in range(200):
        d = np.float64(b[i, 208:210].view(np.float16)[0])
        sc = b[i, 192:208].view(np.int8).astype(np.float64)
        q = O.q6k_quants(b[i], order).astype(np.float64)
        want = (d * sc[np.arange(256) // 16] * q).astype(np.float32)   # exact product, one rounding
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), i


def _q8k_block(rng):
    x = rng.normal(0, 1, 256).astype(np.float32)
    return O.quant_q8_k(x)


@pytest.mark.parametrize("order", [0, 1])
def test_block_int_brute_force(order):
    rng = np.random.default_rng(5)
    for _ in range(64):
        w = rng.integers(0, 256, 210, dtype=np.uint8)
        w[208:210] = [0x00, 0x3C]                  # d = 1: the dequant is sc*q exactly
        xb = _q8k_block(rng)
        sq = O.dequant_q6k(w, order).astype(np.int64)
        xq = xb[4:260].view(np.int8).astype(np.int64)
        assert O.q6k_block_int(w, xb, order) == int((sq * xq).sum())


@pytest.mark.parametrize("order", [0, 1])
def test_gemv_single_block_and_bounds(order):
    rng = np.random.default_rng(9)
    w = rng.integers(0, 256, 210, dtype=np.uint8)
    w[208:210] = [0x00, 0x3C]
    x = rng.normal(0, 1, 256).astype(np.float32)
    xb = O.quant_q8_k(x)
    xb[:4] = np.array([1.0], np.float32).view(np.uint8)   # dy = 1
    y = O.qmatmul_q6k_q8k(w, xb, 1, 256, order)
    assert y[0] == np.float32(O.q6k_block_int(w, xb, order))
    # full rows: within 9 * nb * 2^-24 * sum|terms| of the exact value
    M, K = 6, 4096
    nb = K // 256
    W = rng.integers(0, 256, (M, nb, 210), dtype=np.uint8)
    W[:, :, 208:210] = np.abs(rng.normal(0, 0.02, (M, nb))).astype(np.float16).view(np.uint8).reshape(M, nb, 2)
    xs = O.quant_q8_k(rng.normal(0, 1, K).astype(np.float32))
    y = O.qmatmul_q6k_q8k(W.reshape(-1), xs, M, K, order)
    for r in range(M):
        terms = []
        for b in range(nb):
            d = np.float64(W[r, b, 208:210].view(np.float16)[0])
            dy = np.float64(xs[b * 292: b * 292 + 4].view(np.float32)[0])
            terms.append(d * dy * O.q6k_block_int(W[r, b], xs[b * 292:(b + 1) * 292], order))
        exact = sum(terms)
        assert abs(float(y[r]) - exact) <= 9 * nb * 2.0 ** -24 * sum(abs(t) for t in terms) + 1e-30


def test_mt_wrapper_matches():
    rng = np.random.default_rng(11)
    M, K = 37, 1024
    W = rng.integers(0, 256, M * (K // 256) * 210, dtype=np.uint8)
    xs = O.quant_q8_k(rng.normal(0, 1, K).astype(np.float32))
    for order in (0, 1):
        a = O.qmatmul_q6k_q8k(W, xs, M, K, order)
        b = O.qmatmul_q6k_q8k(W, xs, M, K, order, nthreads=5)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
