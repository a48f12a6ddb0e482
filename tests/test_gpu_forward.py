"""GPU parity of the reference's CPU transformer ABI (include/bpdq_llama.h):
bpd_llama_block_gpu / _s_gpu against the reference's own bpd_llama_block_cpu,
and bpd_llama_forward_gpu / _s_gpu against its bpd_llama_forward_cpu, both
compiled from bench/bpd_cpu.c into oracle/_ref (the -mavx -mssse3 build for
the tile order T, the -O2 build for order S).  Cases: several tokens with
pos_ids and kv_pos > 0 (prefill into a partly filled cache), binary16 and fp32
caches, rope_dim < head_dim, rope_freqs, GQA groups of 1, 2 and 8, contexts
past 1,024 rows.  Bar: bit-exact (x, logits, tokens and both caches)."""
import numpy as np
import pytest
import torch

from bpd_substrate_amd import llama, synth
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LAYER = ("attn_norm_w", "w_q", "w_k", "w_v", "w_o", "ffn_norm_w", "w_gate", "w_up", "w_down")


def config(L=2, E=256, H=4, HKV=2, D=64, F=512, V=300, S=64, rope_dim=None, f16=1, eps=1e-5, base=10000.0):
    return dict(n_layers=L, n_heads=H, n_kv_heads=HKV, head_dim=D, embed_dim=E, ffn_dim=F, vocab_size=V,
                max_seq_len=S, rms_eps=eps, rope_base=base, rope_dim=rope_dim or D, kv_cache_f16=f16)


def make_layer(cfg, key):
    E, H, HKV, D, F = (cfg[n] for n in ("embed_dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim"))
    shapes = {"w_q": (H * D, E), "w_k": (HKV * D, E), "w_v": (HKV * D, E), "w_o": (E, H * D),
              "w_gate": (F, E), "w_up": (F, E), "w_down": (E, F)}
    lw = {"attn_norm_w": (1 + 0.1 * synth.normal_f32(E, synth.key(key, 1))).astype(np.float32),
          "ffn_norm_w": (1 + 0.1 * synth.normal_f32(E, synth.key(key, 2))).astype(np.float32)}
    for i, (n, (r, k)) in enumerate(shapes.items()):
        lw[n] = synth.q8_0(r, k, synth.key(key, 10 + i), d_sigma=0.002)
    return lw


def make_model(cfg, seed, freqs=False):
    E, V = cfg["embed_dim"], cfg["vocab_size"]
    w = {"layers": [make_layer(cfg, 1000 * seed + l) for l in range(cfg["n_layers"])],
         "token_embd": synth.q8_0(V, E, synth.key(seed, 90), d_sigma=0.02),
         "output_norm_w": (1 + 0.1 * synth.normal_f32(E, synth.key(seed, 91))).astype(np.float32),
         "output_w": synth.q8_0(V, E, synth.key(seed, 92), d_sigma=0.002),
         "rope_freqs": None}
    if freqs:   # NTK-style factors >= 1, as Llama 3's rope_freqs.weight
        n = cfg["rope_dim"] // 2
        w["rope_freqs"] = (1.0 + 7.0 * np.abs(synth.normal_f32(n, synth.key(seed, 93)))).astype(np.float32)
    return w


def cache_rows(cfg, n_layers, fill_rows, key):
    """Caches of n_layers layers whose rows 0..fill_rows-1 hold finite data (the
    same on both sides), the rest zero: uint16 bits or fp32."""
    row = cfg["n_kv_heads"] * cfg["head_dim"]
    S = cfg["max_seq_len"]
    out = []
    for which in range(2):
        vals = np.zeros((n_layers, S, row), np.float32)
        vals[:, :fill_rows] = synth.normal_f32(n_layers * fill_rows * row, synth.key(key, which)).reshape(
            n_layers, fill_rows, row)
        out.append(vals.astype(np.float16).view(np.uint16).reshape(-1).copy() if cfg["kv_cache_f16"]
                   else vals.reshape(-1))
    return out


def _d(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dev_cache(a):
    return _d(a.view(np.int16) if a.dtype == np.uint16 else a)


def _host_cache(t, f16):
    a = to_np(t)
    return a.view(np.uint16) if f16 else a


@pytest.mark.parametrize("kind", ["avx", "scalar"])
@pytest.mark.parametrize("f16", [1, 0])
@pytest.mark.parametrize("rope", ["full", "half_freqs"])
@pytest.mark.parametrize("T,kv_pos", [(1, 0), (4, 0), (3, 5), (7, 20)])
def test_block_equals_reference(kind, f16, rope, T, kv_pos):
    cfg = config(L=1, rope_dim=32 if rope == "half_freqs" else None, f16=f16)
    w = make_model(cfg, seed=T + 3 * kv_pos, freqs=rope == "half_freqs")
    lw = w["layers"][0]
    E, F = cfg["embed_dim"], cfg["ffn_dim"]
    x = synth.normal_f32(T * E, synth.key(50, T))
    pos = np.arange(kv_pos, kv_pos + T, dtype=np.int32)
    kc, vc = cache_rows(cfg, 1, kv_pos, 51 + kv_pos)
    xr, kr, vr = x.copy(), kc.copy(), vc.copy()
    if not O.ref_block(lw, cfg, xr, pos, kv_pos, kr, vr, w["rope_freqs"], kind):
        pytest.skip("oracle/_ref not built")
    print(f"block {kind} f16={f16} {rope} T={T} kv_pos={kv_pos}", flush=True)
    dl = {n: _d(lw[n]) for n in LAYER}
    s = llama.layer_struct(dl)
    c = llama.BpdLlamaConfig(*(cfg[n] for n, _ in llama.BpdLlamaConfig._fields_))
    xd, kd, vd = _d(x), _dev_cache(kc), _dev_cache(vc)
    sc = [torch.zeros(T * max(E, F), device="cuda") for _ in range(3)]
    fr = w["rope_freqs"]
    import ctypes
    from bpd_substrate_amd import gpu
    gpu._use_torch_stream()
    gpu.call("bpd_llama_block_s_gpu" if kind == "scalar" else "bpd_llama_block_gpu", xd, ctypes.addressof(s),
             ctypes.addressof(c), pos.ctypes.data, T, kv_pos, kd, vd, sc[0], sc[1], sc[2],
             None if fr is None else fr.ctypes.data)
    torch.cuda.synchronize()
    assert_bits_equal(to_np(xd), xr, "x after the block")
    assert np.array_equal(_host_cache(kd, f16), kr), "K cache"
    assert np.array_equal(_host_cache(vd, f16), vr), "V cache"


def _dev_model(w, cfg):
    dl = [{n: _d(lw[n]) for n in LAYER} for lw in w["layers"]]
    return llama.Forward(cfg, dl, _d(w["token_embd"]), _d(w["output_norm_w"]), _d(w["output_w"]),
                         rope_freqs=w["rope_freqs"], device=torch.device("cuda"))


@pytest.mark.parametrize("kind", ["avx", "scalar"])
@pytest.mark.parametrize("shape", [dict(), dict(H=8, HKV=8, D=32, rope_dim=16),
                                   dict(L=1, E=512, H=4, HKV=1, D=128, F=1024, V=500)])
@pytest.mark.parametrize("freqs", [False, True])
def test_forward_equals_reference(kind, shape, freqs):
    """A 6-token prefill, then two one-token steps, through both forwards with
    binary16 caches (the reference driver's default layout): logits, tokens
    and both caches after every call."""
    cfg = config(**shape)
    w = _forward_case(cfg, kind, freqs, [(6, 0), (1, 6), (1, 7)])


def _forward_case(cfg, kind, freqs, calls, fill=0, seed=11):
    w = make_model(cfg, seed=seed, freqs=freqs)
    kc, vc = cache_rows(cfg, cfg["n_layers"], fill, 60)
    m = _dev_model(w, cfg)
    m.k_cache.copy_(_dev_cache(kc))
    m.v_cache.copy_(_dev_cache(vc))
    order = "S" if kind == "scalar" else "T"
    for i, (T, kv_pos) in enumerate(calls):
        ids = (synth.random_bytes(T * 4, synth.key(70, i)).view(np.uint32) % cfg["vocab_size"]).astype(np.int32)
        pos = np.arange(kv_pos, kv_pos + T, dtype=np.int32)
        print(f"forward {kind} {cfg['embed_dim']}x{cfg['n_heads']}/{cfg['n_kv_heads']} T={T} kv_pos={kv_pos}",
              flush=True)
        want = O.ref_forward(w, cfg, ids, pos, kv_pos, kc, vc, kind)
        if want is None:
            pytest.skip("oracle/_ref not built")
        logits, toks = m.forward(ids, pos, kv_pos, order)
        torch.cuda.synchronize()
        assert_bits_equal(to_np(logits).reshape(T, -1), want[0], f"logits, call {i}")
        assert np.array_equal(to_np(toks), want[1]), f"tokens, call {i}"
        f16 = cfg["kv_cache_f16"]
        assert np.array_equal(_host_cache(m.k_cache, f16), kc), f"K caches, call {i}"
        assert np.array_equal(_host_cache(m.v_cache, f16), vc), f"V caches, call {i}"
    return w


@pytest.mark.parametrize("kind", ["avx", "scalar"])
def test_forward_long_context(kind):
    """Queries at positions 1,100-1,102 over a binary16 cache whose rows below
    1,100 hold random data: the scores span 18 row blocks and P.V streams V in
    128-row chunks."""
    cfg = config(L=1, E=256, H=4, HKV=2, D=64, F=256, V=128, S=2048)
    _forward_case(cfg, kind, True, [(3, 1100)], fill=1100)


@pytest.mark.parametrize("kind", ["avx", "scalar"])
def test_forward_attention_in_token_chunks(kind):
    """300 tokens at positions 7,800-8,099 over a binary16 cache whose first 7,800 rows
    hold random data: the scores of one attention launch are capped at 64 MiB (8 heads x
    8,128 rows x 4 bytes per token: 258 tokens), so the batch's attention runs in two
    launches of the tile kernels, the second at kv_pos + 258."""
    cfg = config(L=1, E=256, H=8, HKV=2, D=32, F=256, V=128, S=8192)
    _forward_case(cfg, kind, False, [(300, 7800)], fill=7800)


def test_forward_fp32_cache_tokens():
    """fp32 caches: bpd_llama_forward_cpu steps between layers by half an fp32
    layer (its uint16_t pointer arithmetic), so only logits and tokens are
    compared, at positions below max_seq_len / 2 where the layouts agree."""
    cfg = config(f16=0)
    w = make_model(cfg, seed=12)
    kc, vc = cache_rows(cfg, cfg["n_layers"], 0, 61)
    m = _dev_model(w, cfg)
    for T, kv_pos in [(5, 0), (1, 5)]:
        ids = np.arange(3, 3 + T, dtype=np.int32)
        pos = np.arange(kv_pos, kv_pos + T, dtype=np.int32)
        want = O.ref_forward(w, cfg, ids, pos, kv_pos, kc, vc, "avx")
        if want is None:
            pytest.skip("oracle/_ref not built")
        logits, toks = m.forward(ids, pos, kv_pos)
        torch.cuda.synchronize()
        assert_bits_equal(to_np(logits).reshape(T, -1), want[0], "logits")
        assert np.array_equal(to_np(toks), want[1])


@pytest.mark.parametrize("order", ["T", "S"])
def test_prefill_equals_stepwise(order):
    """The last row of a 9-token prefill equals 8 tokens of prefill and then one
    step at kv_pos 8 (finite data: every tile of order T gives a cell the same
    bits, and order S is per cell), and so do the caches."""
    cfg = config()
    w = make_model(cfg, seed=13, freqs=True)
    ids = np.arange(10, 19, dtype=np.int32)
    a, b = _dev_model(w, cfg), _dev_model(w, cfg)
    la, ta = a.forward(ids, np.arange(9), 0, order)
    b.forward(ids[:8], np.arange(8), 0, order)
    lb, tb = b.forward(ids[8:], np.array([8]), 8, order)
    torch.cuda.synchronize()
    assert_bits_equal(to_np(la).reshape(9, -1)[8], to_np(lb), "last logits row")
    assert int(to_np(ta)[8]) == int(to_np(tb)[0])
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache)


@pytest.mark.parametrize("kind", ["avx", "scalar"])
@pytest.mark.parametrize("shape,calls,fill", [
    (dict(S=256), [(130, 0)], 0),
    (dict(H=8, HKV=2, D=32, S=256), [(70, 100), (1, 170)], 100),
    (dict(L=1, E=512, H=4, HKV=1, D=128, F=512, V=200, S=256), [(65, 0)], 0)])
def test_forward_token_blocks(kind, shape, calls, fill):
    """Batches past one 64-token softmax / P.V block and one 16-token score tile,
    from an empty cache and into a filled one (rows past a token's own but inside
    its block's tile; chunks where every token of the block has all 64 rows and
    chunks where only some have)."""
    cfg = config(**shape)
    _forward_case(cfg, kind, False, calls, fill=fill)
