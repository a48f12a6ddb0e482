"""GPU parity of the decode step (include/bpdq_llama.h) through the C ABI.

* bpd_expf_gpu equals libm's expf on a strided sweep of all binary32 inputs;
* bpd_residual_rmsnorm_gpu equals the reference's rmsnorm (and the Q8_0
  quantizer) bit-for-bit, including the input whose parallel sum disagrees
  with the sequential one;
* generate_token, with Q8_0 weights in the padded layout, equals the
  reference's own bpd_llama_block_cpu composition from oracle/_ref bit-for-bit
  (token, logits, x, h, K/V caches) step after step, for several GQA shapes;
* the fp32 head, q/k/v biases, long contexts and the Q4_K formats equal the
  restatement bpdq_o_llama_step bit-for-bit.
Bar: bit-exact everywhere.
"""
import numpy as np
import pytest
import torch

import llama_model as LM
from bpd_substrate_amd import gpu, llama
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _d(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_expf_sweep(dev):
    u = np.arange(0, 2 ** 32, 251, dtype=np.uint64).astype(np.uint32)
    # the special-case boundaries: +-Inf, +-0, the overflow / underflow thresholds
    # and |x| = 88 (the start of the special range) with their neighbours
    edges = np.array([0x7f800000, 0xff800000, 0, 0x80000000, 0x42b17218, 0xc2cff1b5, 0x42b00000, 0xc2b00000,
                      0x7f7fffff, 0xff7fffff, 0x00000001, 0x80000001], dtype=np.int64)
    u = np.concatenate([u, (edges[:, None] + np.arange(-2, 3)[None, :]).reshape(-1).astype(np.uint32)])
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    want = O.libm_expf(x)
    y = torch.empty(x.size, dtype=torch.float32, device=dev)
    gpu._use_torch_stream()
    gpu.call("bpd_expf_gpu", _d(x, dev), y, x.size)
    assert_bits_equal(to_np(y), want, "expf")


def _norm(dev, x, add, w, eps, with_q):
    n = x.size
    xo = torch.empty(n, dtype=torch.float32, device=dev)
    h = torch.empty(n, dtype=torch.float32, device=dev)
    xq = torch.empty(n // 32 * 34, dtype=torch.uint8, device=dev) if with_q else None
    gpu._use_torch_stream()
    gpu.call("bpd_residual_rmsnorm_gpu", _d(x, dev), None if add is None else _d(add, dev), xo, _d(w, dev), h, xq,
             n, float(eps))
    torch.cuda.synchronize()
    return to_np(xo), to_np(h), None if xq is None else to_np(xq)


@pytest.mark.parametrize("n", [32, 64, 1024, 4096, 14336, 16384])
def test_residual_rmsnorm(dev, n):
    x = LM.synth.normal_f32(n, LM.synth.key(21, n)) * 2.0
    a = LM.synth.normal_f32(n, LM.synth.key(22, n))
    w = LM._norm_w(n, LM.synth.key(23, n))
    xo, h, xq = _norm(dev, x, a, w, 1e-5, True)
    s = x + a
    assert_bits_equal(xo, s, "residual")
    want = O.rmsnorm(s, w, 1e-5)
    assert_bits_equal(h, want, f"rmsnorm n={n}")
    assert np.array_equal(xq, O.quant_q8_0(want)), "Q8_0 of the normed row"


def test_rmsnorm_sequential_fallback(dev):
    from test_oracle_llama import rmsnorm_hard_case

    x = rmsnorm_hard_case()
    for w in (np.ones(64, np.float32), LM._norm_w(64, LM.synth.key(24, 1))):
        _, h, _ = _norm(dev, x, None, w, 0.0, False)
        assert_bits_equal(h, O.rmsnorm(x, w, 0.0), "rmsnorm hard case")
    # the same case inside a long row, several times over
    big = np.tile(x, 64)
    w = LM._norm_w(big.size, LM.synth.key(24, 2))
    _, h, _ = _norm(dev, big, None, w, 1e-6, False)
    assert_bits_equal(h, O.rmsnorm(big, w, 1e-6), "rmsnorm hard case x64")


def _gpu_model(cfg, layers, head, fmt, dev):
    dl, on, lm, lmf = LM.to_device(cfg, layers, head, fmt, dev)
    return llama.DecodeModel(cfg, dl, on, lm_head=lm, lm_f32=lmf, fmt=fmt, device=dev)


def _check_step(m, got_tok, want, l_caches, pos, what):
    tok, x, h, logits = want
    assert got_tok == tok, f"{what}: token {got_tok} != {tok} at position {pos}"
    assert_bits_equal(to_np(m.buf_t["logits"]), logits, f"{what} logits at {pos}")
    assert_bits_equal(to_np(m.buf_t["x"]), x, f"{what} x at {pos}")
    assert_bits_equal(to_np(m.buf_t["h"]), h, f"{what} h at {pos}")
    kc, vc = l_caches
    for l in range(len(kc)):
        assert_bits_equal(to_np(m.k_cache[l]), kc[l], f"{what} K cache layer {l}")
        assert_bits_equal(to_np(m.v_cache[l]), vc[l], f"{what} V cache layer {l}")


@pytest.mark.parametrize("shape", [dict(), dict(H=8, HKV=8, D=32), dict(H=4, HKV=1, D=128, E=512, F=256),
                                   dict(H=2, HKV=1, D=256, E=512, F=1024, L=3)])
def test_generate_token_equals_reference_block(dev, shape):
    cfg = LM.config(**shape)
    layers, head = LM.make(cfg, 0, seed=3)
    m = _gpu_model(cfg, layers, head, llama.W_Q8_PAD64, dev)
    kr, vr = LM.caches(cfg)
    for pos, e in enumerate(LM.embeddings(cfg, 6)):
        print(f"generate_token {shape} position {pos}", flush=True)
        want = O.ref_llama_step(layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], cfg["vocab_size"])
        if want is None:
            pytest.skip("oracle/_ref not built")
        tok = m.step(_d(e, dev), pos)
        _check_step(m, tok, want, (kr, vr), pos, "generate_token")


@pytest.mark.parametrize("fmt", [llama.W_Q8_PAD64, llama.W_Q4K, llama.W_Q4K_GGUF])
@pytest.mark.parametrize("variant", ["plain", "bias", "f32_head"])
def test_step_equals_restatement(dev, fmt, variant):
    cfg = LM.config(L=2)
    layers, head = LM.make(cfg, fmt, seed=4, bias=variant == "bias", f32_head=variant == "f32_head")
    m = _gpu_model(cfg, layers, head, fmt, dev)
    ko, vo = LM.caches(cfg)
    for pos, e in enumerate(LM.embeddings(cfg, 4, seed=8)):
        print(f"step fmt={fmt} {variant} position {pos}", flush=True)
        want = O.llama_step(fmt, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], head["lm_f32"],
                            cfg["vocab_size"])
        tok = m.step(_d(e, dev), pos)
        _check_step(m, tok, want, (ko, vo), pos, f"fmt {fmt} {variant}")


@pytest.mark.parametrize("fmt", [llama.W_Q4K, llama.W_Q4K_GGUF])
def test_step_wide_embedding(dev, fmt):
    """n_embd = 4096: Q/K/V from the norm's Q8_K, O and gate/up + SwiGLU take the
    K = 4096 span kernels."""
    cfg = LM.config(E=4096, H=32, HKV=8, D=128, F=512, L=1, vocab=300, max_seq=8)
    layers, head = LM.make(cfg, fmt, seed=6)
    m = _gpu_model(cfg, layers, head, fmt, dev)
    ko, vo = LM.caches(cfg)
    for pos, e in enumerate(LM.embeddings(cfg, 2, seed=9)):
        print(f"step fmt={fmt} n_embd=4096 position {pos}", flush=True)
        want = O.llama_step(fmt, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], head["lm_f32"],
                            cfg["vocab_size"])
        tok = m.step(_d(e, dev), pos)
        _check_step(m, tok, want, (ko, vo), pos, f"fmt {fmt} n_embd=4096")


@pytest.mark.parametrize("D,pos,H,HKV,bias", [
    (64, 63, 4, 2, False), (64, 64, 4, 2, False), (64, 255, 4, 2, False), (64, 2047, 4, 2, False),
    (128, 63, 4, 2, False), (128, 300, 4, 2, False), (256, 40, 4, 2, False), (32, 1000, 4, 2, False),
    (64, 1023, 4, 2, False), (128, 1100, 4, 2, False), (32, 16383, 4, 2, False), (32, 16500, 4, 2, False),
    # q/k/v biases; GQA groups of 1 and of 16 (the scores kernel's waves then loop over heads)
    (64, 300, 4, 2, True), (32, 200, 4, 4, False), (32, 130, 16, 1, True)])
def test_long_context(dev, D, pos, H, HKV, bias):
    """Rows 0..pos-1 of the caches hold the same random finite data on both
    sides; one step at `pos` then attends over pos+1 rows (one attention kernel
    up to 64 rows for head_dim <= 128, the scores + P.V pair beyond, whose P.V
    streams V in 128-row chunks for 1024..16384 rows and 64-row chunks
    otherwise; the cases cover whole and partial last chunks of both)."""
    cfg = LM.config(L=1, max_seq=max(2048, pos + 1), E=H * D, H=H, HKV=HKV, D=D)
    layers, head = LM.make(cfg, 0, seed=5, bias=bias)
    m = _gpu_model(cfg, layers, head, llama.W_Q8_PAD64, dev)
    ko, vo = LM.caches(cfg)
    row = cfg["n_head_kv"] * cfg["head_dim"]
    for l in range(cfg["n_layers"]):
        ko[l][:pos * row] = LM.synth.normal_f32(pos * row, LM.synth.key(31, l))
        vo[l][:pos * row] = LM.synth.normal_f32(pos * row, LM.synth.key(32, l))
        m.k_cache[l].copy_(_d(ko[l], dev))
        m.v_cache[l].copy_(_d(vo[l], dev))
    e = LM.embeddings(cfg, 1, seed=9)[0]
    want = O.llama_step(0, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], None, cfg["vocab_size"])
    tok = m.step(_d(e, dev), pos)
    _check_step(m, tok, want, (ko, vo), pos, "long context")


def test_rejects_bad_config(dev):
    cfg = LM.config()
    layers, head = LM.make(cfg, 0, seed=6)
    m = _gpu_model(cfg, layers, head, llama.W_Q8_PAD64, dev)
    e = _d(LM.embeddings(cfg, 1)[0], dev)
    with pytest.raises(gpu.BpdqError, match="position"):
        m.step(e, cfg["max_seq"])
    m.layers[1].down_N = 128
    with pytest.raises(gpu.BpdqError, match="layer 1 down"):
        m.step(e, 0)


@pytest.mark.parametrize("fmt", [llama.W_Q8_PAD64, llama.W_Q4K])
def test_step_norm_fallback_row(dev, fmt):
    """An embedding whose squares sum differently in a tree and in sequence
    (x_0^2/n a binary32 midpoint, 255 squares of 2^-54): layer 0's RMSNorm must
    take the sequential fallback of the norm kernel, with either weight format."""
    cfg = LM.config(L=1)
    e = np.full(cfg["n_embd"], 2.0 ** -27, np.float32)
    e[0] = 1 + 2.0 ** -12
    # every kernel's bound check fails here: (S -+ E)/n straddle an fp32 rounding boundary
    S = float(np.sum(e.astype(np.float64) ** 2))
    E = S * 4 * e.size * 2.0 ** -53
    assert np.float32((S - E) / e.size) != np.float32((S + E) / e.size)
    layers, head = LM.make(cfg, fmt, seed=12)
    for lw in layers:
        lw["attn_norm"] = np.ones(cfg["n_embd"], np.float32)
    m = _gpu_model(cfg, layers, head, fmt, dev)
    ko, vo = LM.caches(cfg)
    want = O.llama_step(fmt, layers, cfg, ko, vo, 0, e, head["out_norm"], head["lm"], None, cfg["vocab_size"])
    tok = m.step(_d(e, dev), 0)
    _check_step(m, tok, want, (ko, vo), 0, f"fallback row fmt {fmt}")


@pytest.mark.parametrize("n", [1, 3, 4, 7, 1000, 4097, 32000, 128256])
def test_argmax_equals_reference(dev, n):
    rng = np.random.default_rng(n)
    cases = [rng.normal(0, 1, n).astype(np.float32), np.zeros(n, np.float32),
             np.round(rng.normal(0, 2, n)).astype(np.float32)]        # many ties
    x = rng.normal(0, 1, n).astype(np.float32)
    x[rng.integers(0, n, max(1, n // 10))] = np.nan                  # NaNs anywhere
    cases.append(x)
    x = cases[0].copy()
    x[0] = np.nan                                                     # NaN first: index 0
    cases.append(x)
    x = -np.zeros(n, np.float32)
    x[n // 2] = 0.0                                                   # +0 does not beat -0
    cases.append(x)
    x = np.full(n, -np.inf, np.float32)
    x[-1] = -1e30                                                     # last element, tail lane
    cases.append(x)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    for i, x in enumerate(cases):
        gpu._use_torch_stream()
        gpu.call("bpd_argmax_gpu", _d(x, dev), n, out)
        assert int(out.item()) == O.argmax(x), (n, i)


def test_captured_step_survives_workspace_growth(dev):
    """A decode step captured in a HIP graph holds the address of its stream's
    workspace.  A later, larger llamafile call on the same stream grows that
    workspace; the buffer the graph holds must stay allocated, so replays still
    give the eager bits and write into no memory allocated since.  After
    bpd_gpu_workspace_release the stream allocates afresh and steps as before."""
    cfg = LM.config(L=2)
    layers, head = LM.make(cfg, 0, seed=13)
    m = _gpu_model(cfg, layers, head, llama.W_Q8_PAD64, dev)
    e = _d(LM.embeddings(cfg, 1, seed=14)[0], dev)
    mw, mt, K = 64, 64, 16384                  # X's Q8_0 rows: 1,114,112 B, above the step's 1 MiB
    W = _d(LM.synth.q8_0(mw, K, LM.synth.key(70, 1)), dev)
    Xh = LM.synth.normal_f32(mt * K, LM.synth.key(70, 2))
    X = _d(Xh, dev)
    s = torch.cuda.Stream()
    try:
        with torch.cuda.stream(s):
            print("workspace growth: eager step on a new stream", flush=True)
            m.enqueue(e, 0)
            s.synchronize()
            want_logits = to_np(m.buf_t["logits"]).copy()
            want_tok = int(m.buf_t["argmax_result"][0].item())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                m.enqueue(e, 0)
            print("workspace growth: larger llamafile call on the same stream", flush=True)
            out = torch.zeros(mt * mw, device=dev)
            gpu._use_torch_stream()
            gpu.call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, out, mw, mt, K)
            s.synchronize()
            assert_bits_equal(to_np(out), O.qmatmul_q8_0_llamafile(LM.synth.q8_0(mw, K, LM.synth.key(70, 1)), Xh,
                                                                    mw, mt, K), "llamafile after growth")
            guard = [torch.full((1 << 18,), 7.0, device=dev) for _ in range(8)]   # 8 x 1 MiB, allocated since
            torch.cuda.synchronize()
            for rep in range(3):
                print(f"workspace growth: replay {rep}", flush=True)
                m.buf_t["logits"].zero_()
                m.buf_t["argmax_result"].fill_(-1)
                g.replay()
                s.synchronize()
                assert_bits_equal(to_np(m.buf_t["logits"]), want_logits, f"replayed step {rep}")
                assert int(m.buf_t["argmax_result"][0].item()) == want_tok
                assert all(bool((t == 7.0).all()) for t in guard), "a replay wrote into memory allocated later"
            del g
        torch.cuda.synchronize()
        gpu.lib().bpd_gpu_set_stream(None)
        gpu.call("bpd_gpu_workspace_release", s.cuda_stream)
        with torch.cuda.stream(s):
            print("workspace growth: eager step after release", flush=True)
            m.buf_t["logits"].zero_()
            m.enqueue(e, 0)
            s.synchronize()
            assert_bits_equal(to_np(m.buf_t["logits"]), want_logits, "step after release")
    finally:
        torch.cuda.synchronize()
        gpu.lib().bpd_gpu_set_stream(None)
        gpu.lib().bpd_gpu_workspace_release(s.cuda_stream)


# ---------------------------------------------------------------- the extended step

def _ext_model(cfg, layers, head, fmt, dev, **kw):
    dl, on, lm, lmf = LM.to_device(cfg, layers, head, fmt, dev)
    return llama.DecodeModel(cfg, dl, on, lm_head=lm, lm_f32=lmf, fmt=fmt, device=dev, **kw)


def _cache_np(t, f16):
    a = to_np(t)
    return a.view(np.uint16) if f16 else a


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("rope", ["full", "half_freqs"])
@pytest.mark.parametrize("shape", [dict(), dict(H=8, HKV=8, D=32), dict(H=4, HKV=1, D=128, E=512, F=256)])
def test_step_ext_equals_reference_block(dev, f16, rope, shape):
    """bpd_llama_step_ext_gpu with padded Q8 weights against the reference's own
    bpd_llama_block_cpu (oracle/_ref, AVX build) with cfg->kv_cache_f16, rope_dim
    and rope_freqs: token, logits, residual, normed row and both caches, 6 steps."""
    cfg = LM.config(**shape)
    D = cfg["head_dim"]
    rd = D // 2 if rope == "half_freqs" else None
    fr = (1.0 + 5.0 * np.abs(LM.synth.normal_f32((rd or D) // 2, LM.synth.key(80, D)))).astype(np.float32) \
        if rope == "half_freqs" else None
    layers, head = LM.make(cfg, 0, seed=15)
    m = _ext_model(cfg, layers, head, llama.W_Q8_PAD64, dev, rope_dim=rd, rope_freqs=fr, kv_cache_f16=f16)
    kr, vr = LM.caches(cfg, f16)
    for pos, e in enumerate(LM.embeddings(cfg, 6, seed=16)):
        print(f"step ext {shape} f16={f16} {rope} position {pos}", flush=True)
        want = O.ref_llama_step(layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], cfg["vocab_size"],
                                rope_dim=rd, rope_freqs=fr, kv_f16=f16)
        if want is None:
            pytest.skip("oracle/_ref not built")
        tok = m.step(_d(e, dev), pos)
        tk, x, h, logits = want
        assert tok == tk, f"token at {pos}"
        assert_bits_equal(to_np(m.buf_t["logits"]), logits, f"logits at {pos}")
        assert_bits_equal(to_np(m.buf_t["x"]), x, f"x at {pos}")
        assert_bits_equal(to_np(m.buf_t["h"]), h, f"h at {pos}")
        for l in range(cfg["n_layers"]):
            assert np.array_equal(_cache_np(m.k_cache[l], f16), kr[l]), f"K cache layer {l} at {pos}"
            assert np.array_equal(_cache_np(m.v_cache[l], f16), vr[l]), f"V cache layer {l} at {pos}"


@pytest.mark.parametrize("D,pos", [(64, 63), (64, 200), (128, 1100), (32, 3000)])
def test_step_ext_long_context_f16(dev, D, pos):
    """Binary16 caches at every attention regime (one-kernel up to 64 rows, scores +
    P.V with 64- and 128-row chunks): rows 0..pos-1 hold the same random binary16
    data on both sides, one step at pos against the reference block."""
    H, HKV = 4, 2
    cfg = LM.config(L=1, max_seq=max(2048, pos + 1), E=H * D, H=H, HKV=HKV, D=D)
    layers, head = LM.make(cfg, 0, seed=17)
    m = _ext_model(cfg, layers, head, llama.W_Q8_PAD64, dev, kv_cache_f16=True)
    kr, vr = LM.caches(cfg, True)
    row = HKV * D
    for l in range(cfg["n_layers"]):
        kr[l][:pos * row] = LM.synth.normal_f32(pos * row, LM.synth.key(81, l)).astype(np.float16).view(np.uint16)
        vr[l][:pos * row] = LM.synth.normal_f32(pos * row, LM.synth.key(82, l)).astype(np.float16).view(np.uint16)
        m.k_cache[l].copy_(_d(kr[l].view(np.int16), dev))
        m.v_cache[l].copy_(_d(vr[l].view(np.int16), dev))
    e = LM.embeddings(cfg, 1, seed=18)[0]
    want = O.ref_llama_step(layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], cfg["vocab_size"], kv_f16=True)
    if want is None:
        pytest.skip("oracle/_ref not built")
    tok = m.step(_d(e, dev), pos)
    assert tok == want[0]
    assert_bits_equal(to_np(m.buf_t["logits"]), want[3], "logits")
    assert np.array_equal(_cache_np(m.k_cache[0], True), kr[0]) and np.array_equal(_cache_np(m.v_cache[0], True), vr[0])


Q4KM = {"v": llama.W_Q6K_GGUF, "down": llama.W_Q6K_GGUF}           # what llama.cpp's Q4_K_M keeps in Q6_K


@pytest.mark.parametrize("case", ["q4k_m", "q4k_m_bpd", "q6k_gate", "wide", "f16_rope"])
def test_step_mixed_formats(dev, case):
    """Per-matrix formats: Q4_K with Q6_K attn_v / ffn_down and a Q6_K head (a
    Q4_K_M file), both element maps, a Q6_K gate (gate/up as two GEMVs and
    SwiGLU), n_embd = 8192 (no normed Q8_K row: Q6_K matrices quantize their
    input), and with binary16 caches and rope_freqs; against the restatement
    bpdq_o_llama_step_ext, 3 steps, bit for bit."""
    base, lm_fmt, fm, kw, shape = llama.W_Q4K_GGUF, llama.W_Q6K_GGUF, dict(Q4KM), {}, dict()
    if case == "q4k_m_bpd":
        base, lm_fmt, fm = llama.W_Q4K, llama.W_Q6K, {"v": llama.W_Q6K, "down": llama.W_Q6K}
    elif case == "q6k_gate":
        fm = {"gate": llama.W_Q6K_GGUF, "o": llama.W_Q6K_GGUF}
    elif case == "wide":
        shape = dict(E=8192, H=64, HKV=8, D=128, F=512, L=1, vocab=300, max_seq=8)
    elif case == "f16_rope":
        kw = dict(kv_cache_f16=True, rope_dim=32,
                  rope_freqs=(1.0 + np.arange(16, dtype=np.float32) / 3).astype(np.float32))
    cfg = LM.config(**shape)
    L = cfg["n_layers"]
    formats = [dict(fm) for _ in range(L)]
    if case == "q4k_m" and L > 1:
        formats[1] = {}                      # Q4_K_M keeps Q6_K in some layers only
    layers, head = LM.make(cfg, base, seed=19, formats=formats, lm_fmt=lm_fmt)
    m = _ext_model(cfg, layers, head, base, dev, formats=formats, lm_format=lm_fmt, **kw)
    f16 = kw.get("kv_cache_f16", False)
    ko, vo = LM.caches(cfg, f16)
    fmts = [[formats[l].get(n, base) for n in LM.MATS] for l in range(L)]
    for pos, e in enumerate(LM.embeddings(cfg, 3, seed=20)):
        print(f"mixed formats {case} position {pos}", flush=True)
        want = O.llama_step_ext(fmts, lm_fmt, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], None,
                                cfg["vocab_size"], rope_dim=kw.get("rope_dim"), rope_freqs=kw.get("rope_freqs"),
                                kv_f16=f16)
        tok = m.step(_d(e, dev), pos)
        assert tok == want[0], f"token at {pos}"
        assert_bits_equal(to_np(m.buf_t["logits"]), want[3], f"{case} logits at {pos}")
        assert_bits_equal(to_np(m.buf_t["x"]), want[1], f"{case} x at {pos}")
        for l in range(L):
            assert np.array_equal(_cache_np(m.k_cache[l], f16), ko[l]), f"K cache layer {l}"
            assert np.array_equal(_cache_np(m.v_cache[l], f16), vo[l]), f"V cache layer {l}"


# ---------------------------------------------------------------- RMSNorm folded into the GEMVs

@pytest.mark.parametrize("fmt,F,L", [(llama.W_Q4K, 4096, 3), (llama.W_Q4K_GGUF, 4096, 3),
                                     (llama.W_Q4K_GGUF, 14336, 2)])
def test_step_folded_norms(dev, fmt, F, L):
    """n_embd = 4096, all matrices Q4_K: the O and down GEMVs add into the residual
    row and write partial sums of squares, and the Q/K/V and gate/up GEMVs compute
    the norm themselves (layer 0's attention norm stays a launch of its own).
    Against the restatement bpdq_o_llama_step, 3 steps, bit for bit."""
    cfg = LM.config(E=4096, H=32, HKV=8, D=128, F=F, L=L, vocab=300, max_seq=8)
    layers, head = LM.make(cfg, fmt, seed=23)
    m = _gpu_model(cfg, layers, head, fmt, dev)
    ko, vo = LM.caches(cfg)
    for pos, e in enumerate(LM.embeddings(cfg, 3, seed=24)):
        print(f"folded norms fmt={fmt} F={F} position {pos}", flush=True)
        want = O.llama_step(fmt, layers, cfg, ko, vo, pos, e, head["out_norm"], head["lm"], None, cfg["vocab_size"])
        tok = m.step(_d(e, dev), pos)
        _check_step(m, tok, want, (ko, vo), pos, f"folded norms fmt {fmt} F {F}")


def test_step_folded_norm_fallback(dev):
    """Layer 0's matrices are all zero (d = dmin = 0), so the residual row entering
    layer 1's folded attention norm, and layer 0's folded FFN norm, is the embedding
    itself: a row whose binary64 sum of squares straddles an fp32 rounding boundary
    of the mean, so the folded norms must take the sequential fallback."""
    cfg = LM.config(E=4096, H=32, HKV=8, D=128, F=4096, L=2, vocab=300, max_seq=8)
    n = cfg["n_embd"]
    e = np.full(n, 2.0 ** -27, np.float32)
    e[0] = 1 + 2.0 ** -12
    S = float(np.sum(e.astype(np.float64) ** 2))
    E = S * 4 * n * 2.0 ** -53
    assert np.float32((S - E) / n) != np.float32((S + E) / n)
    layers, head = LM.make(cfg, llama.W_Q4K_GGUF, seed=25)
    for mname in LM.MATS:
        layers[0][mname] = np.zeros_like(layers[0][mname])
    for lw in layers:
        lw["attn_norm"] = np.ones(n, np.float32)
        lw["ffn_norm"] = np.ones(n, np.float32)
    m = _gpu_model(cfg, layers, head, llama.W_Q4K_GGUF, dev)
    ko, vo = LM.caches(cfg)
    want = O.llama_step(llama.W_Q4K_GGUF, layers, cfg, ko, vo, 0, e, head["out_norm"], head["lm"], None,
                        cfg["vocab_size"])
    tok = m.step(_d(e, dev), 0)
    _check_step(m, tok, want, (ko, vo), 0, "folded norm fallback")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("D,pos,H,HKV", [
    (64, 2047, 4, 2), (64, 300, 4, 2), (128, 1100, 4, 2), (128, 1023, 8, 2), (64, 200, 16, 1), (128, 4000, 8, 2)])
def test_long_context_kquant(dev, D, pos, H, HKV, f16):
    """K-quant weights (no Q8_0 attention output): P.V in 16-column slices, whose
    workgroups the (kv head, slice) pairs map onto XCDs when they divide into 8
    (every case here but the single-kv-head one).  One step at pos over
    pos + 1 cached rows, against the reference block."""
    cfg = LM.config(L=1, max_seq=max(2048, pos + 1), E=H * D, H=H, HKV=HKV, D=D, F=256)
    layers, head = LM.make(cfg, llama.W_Q4K, seed=19)
    m = _ext_model(cfg, layers, head, llama.W_Q4K, dev, kv_cache_f16=f16)
    kr, vr = LM.caches(cfg, f16)
    row = HKV * D
    for l in range(cfg["n_layers"]):
        k = LM.synth.normal_f32(pos * row, LM.synth.key(83, l))
        v = LM.synth.normal_f32(pos * row, LM.synth.key(84, l))
        kr[l][:pos * row] = k.astype(np.float16).view(np.uint16) if f16 else k
        vr[l][:pos * row] = v.astype(np.float16).view(np.uint16) if f16 else v
        m.k_cache[l].copy_(_d(kr[l].view(np.int16) if f16 else kr[l], dev))
        m.v_cache[l].copy_(_d(vr[l].view(np.int16) if f16 else vr[l], dev))
    e = LM.embeddings(cfg, 1, seed=20)[0]
    print(f"long context K-quant D={D} pos={pos} H={H} HKV={HKV} f16={f16}", flush=True)
    fmts = [[llama.W_Q4K] * 7 for _ in range(cfg["n_layers"])]
    want = O.llama_step_ext(fmts, llama.W_Q4K, layers, cfg, kr, vr, pos, e, head["out_norm"], head["lm"], None,
                            cfg["vocab_size"], kv_f16=f16)
    tok = m.step(_d(e, dev), pos)
    assert tok == want[0], f"token at {pos}"
    assert_bits_equal(to_np(m.buf_t["logits"]), want[3], f"logits at {pos}")
    assert_bits_equal(to_np(m.buf_t["x"]), want[1], f"x at {pos}")
    assert_bits_equal(to_np(m.buf_t["h"]), want[2], f"h at {pos}")
    for l in range(cfg["n_layers"]):
        assert np.array_equal(_cache_np(m.k_cache[l], f16), kr[l]), f"K cache layer {l}"
        assert np.array_equal(_cache_np(m.v_cache[l], f16), vr[l]), f"V cache layer {l}"
