"""Pins of the decode-step restatement in oracle/bpdq_oracle.c (CPU only).

* expf: the restated libm method equals the C library's expf on every non-NaN
  binary32 input (exhaustive), its table is the correctly rounded 2^(i/32)
  (recomputed here at 200-bit precision), and its special cases are IEEE's;
* each step function equals the reference's compiled function from
  oracle/_ref (bench/bpd_cpu.c: rmsnorm :4959, rope :5146, attention :5370,
  swiglu :5504, argmax :4512), including the edge cases those define;
* the whole step (Q8_0, tile order T) equals the reference's
  bpd_llama_block_cpu composition bit-for-bit over several positions, GQA
  shapes and head dims;
* the fp32 head order (no reference source): exact on integer data, within
  its error bound on random data;
* the RMSNorm input that makes a parallel sum disagree with the reference's
  sequential one exists and is the one the GPU test uses.
"""
import os
import struct

import numpy as np
import pytest

import llama_model as LM
from bpd_substrate_amd import formats
from helpers import assert_bits_equal
from oracle import oracle as O

NEEDS_REF = pytest.mark.skipif(O.ref("avx") is None, reason="oracle/_ref not built (make -C oracle ref)")


def test_expf_equals_libm_on_every_input():
    n, first = O.expf_mismatches(nthreads=os.cpu_count() or 8, stride=1)
    assert n == 0, f"{n} inputs differ, first bits 0x{first:08x}"


def test_expf_table_is_rounded_powers_of_two():
    mpmath = pytest.importorskip("mpmath")
    mpmath.mp.prec = 200
    for i, t in enumerate(O.expf_table()):
        d = float(mpmath.power(2, mpmath.mpf(i) / 32))
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert int(t) == (bits - ((i << 52) // 32)) & (2 ** 64 - 1), i


def test_expf_special_values():
    f = lambda v: O.expf_nagy(v)
    assert f(0.0) == 1.0 and f(-0.0) == 1.0
    assert f(float("inf")) == float("inf") and f(float("-inf")) == 0.0
    assert np.isnan(f(float("nan")))
    assert f(89.0) == float("inf") and f(-104.0) == 0.0
    assert f(88.72) < float("inf")                       # largest finite region
    sub = f(-100.0)
    assert 0 < sub < np.finfo(np.float32).tiny           # subnormal result


def _ref_fn(name, args, res=None):
    import ctypes

    R = O.ref("avx")
    fn = getattr(R, name)
    fn.argtypes, fn.restype = args, res
    return fn


P, I, F = O.P, O.I, O.F


@NEEDS_REF
@pytest.mark.parametrize("n", [32, 256, 4096])
def test_rmsnorm_equals_reference(n):
    rm = _ref_fn("bpd_rmsnorm_llama_cpu", [P, P, P, I, I, F])
    x = LM.synth.normal_f32(n, LM.synth.key(3, n)) * 3.0
    w = LM._norm_w(n, LM.synth.key(4, n))
    want = np.empty(n, np.float32)
    rm(x.ctypes.data, w.ctypes.data, want.ctypes.data, 1, n, 1e-5)
    assert_bits_equal(O.rmsnorm(x, w, 1e-5), want, "rmsnorm")


@NEEDS_REF
@pytest.mark.parametrize("D,pos", [(64, 0), (64, 17), (128, 1000), (256, 31000)])
def test_rope_equals_reference(D, pos):
    rope = _ref_fn("bpd_rope_norm_freqs_cpu", [P, P, P, P, I, I, I, I, F])
    H = 3
    t = LM.synth.normal_f32(H * D, LM.synth.key(5, D + pos))
    want = np.empty_like(t)
    p = np.array([pos], np.int32)
    rope(t.ctypes.data, want.ctypes.data, p.ctypes.data, None, 1, H, D, D, 500000.0)
    assert_bits_equal(O.rope_norm(t, H, D, pos, 500000.0), want, "rope")


@NEEDS_REF
@pytest.mark.parametrize("D,n_dims,pos,freqs", [(64, 32, 17, True), (128, 64, 1000, True), (128, 128, 4000, True),
                                                 (64, 2, 31000, False), (256, 200, 77, True)])
def test_rope_freqs_partial_equals_reference(D, n_dims, pos, freqs):
    """bpdq_o_rope_norm_freqs against bpd_rope_norm_freqs_cpu with frequency factors
    and n_dims < head_dim (the tail of each head passes through)."""
    rope = _ref_fn("bpd_rope_norm_freqs_cpu", [P, P, P, P, I, I, I, I, F])
    H = 3
    t = LM.synth.normal_f32(H * D, LM.synth.key(5, D + pos + n_dims))
    ff = (1.0 + 9.0 * np.abs(LM.synth.normal_f32(n_dims // 2, LM.synth.key(9, n_dims)))).astype(np.float32) \
        if freqs else None
    want = np.empty_like(t)
    p = np.array([pos], np.int32)
    rope(t.ctypes.data, want.ctypes.data, p.ctypes.data, None if ff is None else ff.ctypes.data, 1, H, D, n_dims,
         500000.0)
    got = t.copy()
    O.lib().bpdq_o_rope_norm_freqs(got.ctypes.data, H, D, pos, 500000.0, n_dims,
                                   None if ff is None else ff.ctypes.data)
    assert_bits_equal(got, want, "rope with freqs")
    assert np.array_equal(got.reshape(H, D)[:, n_dims:], t.reshape(H, D)[:, n_dims:])   # the tail unchanged


@NEEDS_REF
@pytest.mark.parametrize("H,HKV,D,S,pos", [(4, 2, 64, 16, 0), (4, 2, 64, 16, 9), (8, 8, 32, 40, 39),
                                           (6, 1, 128, 33, 20)])
def test_attention_equals_reference(H, HKV, D, S, pos):
    att = _ref_fn("bpd_gqa_attn_cpu", [P, P, P, P, I, I, I, I, I, F, I])
    k = LM.synth.key(6, H * 100 + pos)
    q = LM.synth.normal_f32(H * D, k)
    kc = np.zeros(S * HKV * D, np.float32)
    vc = np.zeros(S * HKV * D, np.float32)
    kc[:(pos + 1) * HKV * D] = LM.synth.normal_f32((pos + 1) * HKV * D, k + 1)
    vc[:(pos + 1) * HKV * D] = LM.synth.normal_f32((pos + 1) * HKV * D, k + 2)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    want = np.empty(H * D, np.float32)
    att(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, want.ctypes.data, 1, S, H, HKV, D, float(scale), pos)
    assert_bits_equal(O.gqa_attn(q, kc, vc, S, pos, H, HKV, D, float(scale)), want, "attention")


@NEEDS_REF
def test_swiglu_and_argmax_equal_reference():
    sw = _ref_fn("bpd_swiglu_fuse_cpu", [P, P, P, I])
    am = _ref_fn("bpd_argmax_dim_cpu", [P, P, I, I, I])
    g = LM.synth.normal_f32(4096, LM.synth.key(8, 1)) * 6.0
    g[:4] = [0.0, -0.0, 88.0, -104.0]
    u = LM.synth.normal_f32(4096, LM.synth.key(8, 2))
    want = np.empty_like(g)
    sw(g.ctypes.data, u.ctypes.data, want.ctypes.data, g.size)
    assert_bits_equal(O.swiglu(g, u), want, "swiglu")

    def ref_argmax(x):
        out = np.zeros(1, np.int64)
        am(x.ctypes.data, out.ctypes.data, 1, x.size, 1)
        return int(out[0])

    cases = [np.array([1.0, 3.0, 3.0, 2.0], np.float32),          # first of a tie
             np.array([-0.0, 0.0, -1.0], np.float32),              # +0 does not beat -0
             np.array([np.nan, 5.0, 1.0], np.float32),             # NaN first: index 0
             np.array([1.0, np.nan, 5.0, np.nan], np.float32),     # later NaNs are skipped
             np.array([-np.inf, -np.inf], np.float32),
             LM.synth.normal_f32(5000, LM.synth.key(8, 3))]
    for x in cases:
        assert O.argmax(x) == ref_argmax(x), x[:6]


@NEEDS_REF
@pytest.mark.parametrize("shape", [dict(), dict(H=8, HKV=8, D=32), dict(H=4, HKV=1, D=128, E=512, F=256)])
def test_step_equals_reference_block(shape):
    cfg = LM.config(**shape)
    layers, head = LM.make(cfg, 0, seed=2)
    kr, vr = LM.caches(cfg)
    ko, vo = LM.caches(cfg)
    for pos, e in enumerate(LM.embeddings(cfg, 5)):
        r = O.ref_llama_step(layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], cfg["vocab_size"])
        o = O.llama_step(0, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], None, cfg["vocab_size"])
        assert r[0] == o[0]
        for a, b, what in zip(o[1:], r[1:], ("x", "h", "logits")):
            assert_bits_equal(a, b, f"{what} at position {pos}")
        for l in range(cfg["n_layers"]):
            assert_bits_equal(ko[l], kr[l], "K cache")
            assert_bits_equal(vo[l], vr[l], "V cache")


@NEEDS_REF
@pytest.mark.parametrize("f16,rope", [(True, "full"), (True, "half_freqs"), (False, "half_freqs")])
def test_step_ext_equals_reference_block(f16, rope):
    """The restatement's binary16 caches, rope_dim and frequency factors
    (bpdq_o_llama_step_ext, padded-Q8 weights) against the reference's own
    bpd_llama_block_cpu with cfg->kv_cache_f16, rope_dim and rope_freqs."""
    cfg = LM.config()
    D = cfg["head_dim"]
    rd = D // 2 if rope == "half_freqs" else None
    fr = (1.0 + np.arange((rd or D) // 2, dtype=np.float32) / 2).astype(np.float32) if rd else None
    layers, head = LM.make(cfg, 0, seed=2)
    kr, vr = LM.caches(cfg, f16)
    ko, vo = LM.caches(cfg, f16)
    fm = [[0] * 7 for _ in range(cfg["n_layers"])]
    for pos, e in enumerate(LM.embeddings(cfg, 5)):
        r = O.ref_llama_step(layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], cfg["vocab_size"],
                             rope_dim=rd, rope_freqs=fr, kv_f16=f16)
        o = O.llama_step_ext(fm, 0, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], None,
                             cfg["vocab_size"], rope_dim=rd, rope_freqs=fr, kv_f16=f16)
        assert r[0] == o[0]
        for a, b, what in zip(o[1:], r[1:], ("x", "h", "logits")):
            assert_bits_equal(a, b, f"{what} at position {pos}")
        for l in range(cfg["n_layers"]):
            assert np.array_equal(ko[l], kr[l]) and np.array_equal(vo[l], vr[l]), "caches"


def test_step_ext_q6k_matrices_are_the_q6k_gemv():
    """A K-quant step whose v and down are Q6_K equals, layer by layer, the plain
    composition with bpdq_o_qmatmul_q6k_q8k of the Q8_K activation in those two
    places: the restatement's format dispatch picks the Q6_K product."""
    cfg = LM.config(L=1)
    fm = {"v": 4, "down": 4}
    layers, head = LM.make(cfg, 2, seed=21, formats=[fm], lm_fmt=4)
    e = LM.embeddings(cfg, 1, seed=22)[0]
    ko, vo = LM.caches(cfg)
    tok, x, h, logits = O.llama_step_ext([[fm.get(n, 2) for n in LM.MATS]], 4, layers, cfg, ko, vo, 0, e,
                                         head["out_norm"], head["lm"], None, cfg["vocab_size"])
    lw = layers[0]
    E, F, row = cfg["n_embd"], cfg["ff_dim"], cfg["n_head_kv"] * cfg["head_dim"]
    hh = O.rmsnorm(e, lw["attn_norm"], cfg["eps"])
    v = O.qmatmul_q6k_q8k(lw["v"], O.quant_q8_k(hh), row, E, order=1)
    assert_bits_equal(vo[0][:row], v, "V row 0 = the Q6_K GEMV of the normed embedding")
    assert_bits_equal(logits, O.qmatmul_q6k_q8k(head["lm"], O.quant_q8_k(h), cfg["vocab_size"], E, order=1),
                      "Q6_K head")


def test_gemv_f32_order_pins():
    rng = np.random.default_rng(1)
    N, K = 9, 300
    W = rng.integers(-8, 8, (N, K)).astype(np.float32)
    x = rng.integers(-8, 8, K).astype(np.float32)
    assert np.array_equal(O.gemv_f32_wave(W, x, N, K), (W.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, K).astype(np.float32)
    exact = W.astype(np.float64) @ x.astype(np.float64)
    bound = (K // 64 + 8) * 2.0 ** -24 * (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    assert (np.abs(O.gemv_f32_wave(W, x, N, K) - exact) <= bound).all()


def kernel_tree_mean(x, NT=1024):
    """The binary64 sum of squares as k_residual_rmsnorm forms it without its
    fallback: per-thread strided sums, xor butterfly per 64-lane wave (lane 0
    kept), then the wave sums in order."""
    x = x.astype(np.float64)
    n = x.size
    lanes = np.zeros(NT)
    for t in range(NT):
        s = 0.0
        for i in range(t, n, NT):
            s += x[i] * x[i]
        lanes[t] = s
    total = 0.0
    for w in range(NT // 64):
        v = lanes[64 * w:64 * w + 64].copy()
        for m in (32, 16, 8, 4, 2, 1):
            v = np.array([v[l] + v[l ^ m] for l in range(64)])
        total += v[0]
    return np.float32(total / n)


def rmsnorm_hard_case():
    """x_0^2 / 64 is a binary32 midpoint and 63 squares of 2^-54 vanish one by
    one in the sequential sum but not in a tree."""
    x = np.full(64, 2.0 ** -27, np.float32)
    x[0] = 1 + 2.0 ** -12
    return x


def test_rmsnorm_hard_case_separates_tree_and_sequential():
    x = rmsnorm_hard_case()
    seq = 0.0
    for v in x.astype(np.float64):
        seq += v * v
    assert np.float32(seq / 64) != kernel_tree_mean(x)
    w = np.ones(64, np.float32)
    # the restatement follows the sequential sum
    y = O.rmsnorm(x, w, 0.0)
    assert y[0] == np.float32(x[0] * (np.float32(1) / np.sqrt(np.float32(seq / 64))))


def test_q8_0_rows_to_pad64_is_a_relayout():
    n, k = 5, 96
    rows = LM.synth.q8_0(n, k, LM.synth.key(9, 1))
    pad = formats.q8_0_rows_to_pad64(rows, n, k).reshape(k // 32, n, 64)
    src = rows.reshape(n, k // 32, 34)
    for b in range(k // 32):
        for r in range(n):
            assert bytes(pad[b, r, 0:2]) == bytes(src[r, b, 0:2])
            assert bytes(pad[b, r, 2:4]) == b"\0\0" and not pad[b, r, 36:].any()
            assert bytes(pad[b, r, 4:36]) == bytes(src[r, b, 2:34])
