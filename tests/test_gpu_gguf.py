"""GGUF bytes straight into the GPU ABI: tensors written to a GGUF file, located
by bpd_substrate_amd.gguf, copied to the device unchanged and consumed by the
entry points; outputs compared with the oracle on the bytes read back from the
file."""
import numpy as np
import pytest

from bpd_substrate_amd import gguf, gpu, synth
from helpers import assert_bits_equal, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_gguf_tensors_feed_the_abi(dev, tmp_path):
    import torch

    M, K, V, E = 1024, 4096, 512, 256
    w = synth.q4k(M, K, synth.key(61, 1))
    emb = synth.q8_0(V, E, synth.key(61, 2))
    p = str(tmp_path / "model.gguf")
    gguf.write_gguf(p, [("general.architecture", gguf.T_STR, "llama"), ("llama.rope.freq_base", gguf.T_F32, 1e4),
                        ("general.quantization_version", gguf.T_U32, 3)],
                    [("token_embd.weight", (E, V), gguf.Q8_0, emb.tobytes()),
                     ("blk.0.ffn_gate.weight", (K, M), gguf.Q4_K, w.tobytes())])
    g = gguf.open_gguf(p)
    assert all(ok for _, ok, _ in gguf.report(p))
    t = g.tensor("blk.0.ffn_gate.weight")
    assert (t.row_len, t.n_rows) == (K, M)
    host_w = np.frombuffer(g.tensor_bytes(t.name), np.uint8).copy()
    wd = g.to_device(t.name, dev)
    x = synth.normal_f32(K, synth.key(61, 3))
    y = gpu.qmatmul_q4k_q8k_fused(wd, torch.from_numpy(x).to(dev), M, K)
    assert_bits_equal(to_np(y), O.qmatmul_q4k_q8k(host_w, O.quant_q8_k(x), M, K, 0, nthreads=8), "gguf Q4_K GEMV")
    deq = gpu.dequant_q4k(wd[: 64 * 144])
    assert_bits_equal(to_np(deq), O.dequant_q4k(host_w[: 64 * 144]), "gguf Q4_K dequant")

    e = g.tensor("token_embd.weight")
    ed = g.to_device(e.name, dev)
    ids = torch.tensor([0, 7, V - 1, 7], dtype=torch.int32, device=dev)
    out = gpu.embed_lookup_q8_0(ed, ids, E)
    host_e = np.frombuffer(g.tensor_bytes(e.name), np.uint8).copy()
    want = O.embed_lookup_q8_0(host_e, np.array([0, 7, V - 1, 7], np.int32), E)
    assert_bits_equal(to_np(out).ravel(), want.ravel(), "gguf Q8_0 embedding rows")


# ---------------------------------------------------------------- whole models from GGUF

@pytest.mark.parametrize("case", ["q4k_m", "tied", "q8_0"])
def test_decode_model_from_gguf(dev, tmp_path, case):
    """DecodeModel.from_gguf on a synthetic llama file: a Q4_K_M layout (Q6_K
    attn_v / ffn_down in layer 0 and a Q6_K output.weight, rope_dim and
    rope_freqs.weight), a tied head (token_embd as the head), and an all-Q8_0
    file (padded layout, checked against the reference's own block).  Three
    tokens stepped from their embeddings, bit for bit."""
    import gguf_model as GM
    import llama_model as LM
    from bpd_substrate_amd import llama

    cfg = LM.config(L=2, vocab=300, max_seq=16)
    E, V = cfg["n_embd"], cfg["vocab_size"]
    if case == "q8_0":
        layers, head = LM.make(cfg, 0, seed=33)
        embd = (LM.synth.q8_0(V, E, LM.synth.key(33, 5), d_sigma=0.02), gguf.Q8_0)
        fm, base, lm_fmt, rd, fr = None, 0, 0, None, None
    else:
        fm = [{"v": 4, "down": 4}, {}]
        base, lm_fmt = 2, (2 if case == "tied" else 4)
        layers, head = LM.make(cfg, 2, seed=33, formats=fm, lm_fmt=lm_fmt)
        embd = (LM.synth.q4k(V, E, LM.synth.key(33, 5)), gguf.Q4_K)
        rd, fr = 32, np.linspace(1, 4, 16).astype(np.float32)
        if case == "tied":
            head["lm"] = embd[0]
    path = str(tmp_path / f"{case}.gguf")
    GM.write_model(path, cfg, layers, head, embd, base, fm, lm_fmt, rope_dim=rd, rope_freqs=fr,
                   tied=case == "tied")
    m = llama.DecodeModel.from_gguf(path, dev, max_seq=cfg["max_seq"])
    ko, vo = LM.caches(cfg)
    fmts = [[(fm[l] if fm else {}).get(n, base) for n in LM.MATS] for l in range(cfg["n_layers"])]
    for pos, tok_in in enumerate([5, 17, 299]):
        print(f"from_gguf {case} position {pos}", flush=True)
        emb = m.embed(tok_in)
        nb = E // (256 if embd[1] == gguf.Q4_K else 32)
        bpb = 144 if embd[1] == gguf.Q4_K else 34
        row = embd[0][tok_in * nb * bpb:(tok_in + 1) * nb * bpb]
        want_emb = O.dequant_q4k_gguf(row) if embd[1] == gguf.Q4_K else O.dequant_q8_0(row)
        assert_bits_equal(to_np(emb), want_emb, "embedding row")
        if case == "q8_0":
            want = O.ref_llama_step(layers, cfg, ko, vo, pos, want_emb, head["out_norm"], head["lm"], V)
            if want is None:
                pytest.skip("oracle/_ref not built")
        else:
            want = O.llama_step_ext(fmts, lm_fmt, layers, cfg, ko, vo, pos, want_emb, head["out_norm"], head["lm"],
                                    None, V, rope_dim=rd, rope_freqs=fr)
        tok = m.step(emb, pos)
        assert tok == want[0], f"token at {pos}"
        assert_bits_equal(to_np(m.buf_t["logits"]), want[3], f"{case} logits at {pos}")
        for l in range(cfg["n_layers"]):
            assert_bits_equal(to_np(m.k_cache[l]), ko[l], f"K cache layer {l}")


# ---------------------------------------------------------------- the reference loader

def _pad64_to_q8_0_rows(p, n, k):
    """The inverse relayout of formats.q8_0_rows_to_pad64: [k/32][n][64] -> Q8_0 rows."""
    nb = k // 32
    r = np.asarray(p, np.uint8).reshape(nb, n, 64)
    out = np.zeros((n, nb, 34), np.uint8)
    out[:, :, 0:2] = r[:, :, 0:2].transpose(1, 0, 2)
    out[:, :, 2:34] = r[:, :, 4:36].transpose(1, 0, 2)
    return out.reshape(-1)


# f16 scale offsets of each block type, for realistic (small, finite) scales
_SCALES = {2: (0,), 10: (80, 82), 11: (108,), 12: (0, 2), 14: (208,)}


def _tensor(n_rows, k, code, seed):
    rng = np.random.default_rng(seed)
    if code == 0:
        return rng.normal(0, 0.05, n_rows * k).astype(np.float32).view(np.uint8)
    if code == 1:
        return rng.normal(0, 0.05, n_rows * k).astype(np.float16).view(np.uint8)
    per, size = gpu.GGUF_PY_BLOCKS[code]
    b = rng.integers(0, 256, (n_rows * k // per, size), dtype=np.uint8)
    for o in _SCALES[code]:
        b[:, o:o + 2] = np.abs(rng.normal(0, 0.004, b.shape[0])).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def test_decode_model_reference_loader(dev, tmp_path):
    """A synthetic llama file whose matrices use every type the reference loader
    reads and the native one does not (Q4_0, Q2_K, Q3_K, F16, F32), beside Q4_K and
    Q6_K, with an F32 output.weight and a Q2_K token table.  from_gguf falls back to
    the reference loader. Three checks follow:
    * every padded-Q8 weight on the device equals the oracle's q8_pad64 of the
      oracle's load_tensor_by_type fp32, byte for byte;
    * the embedding rows equal the oracle's fp32 table;
    * three tokens stepped from those rows match the reference's own C block with
      the same weights, bit for bit."""
    import gguf_model as GM
    import llama_model as LM
    from bpd_substrate_amd import llama

    cfg = LM.config(L=2, vocab=300, max_seq=16)
    E, H, HKV, D, F, V = (cfg[n] for n in ("n_embd", "n_head", "n_head_kv", "head_dim", "ff_dim", "vocab_size"))
    rows = {"q": (H * D, E), "k": (HKV * D, E), "v": (HKV * D, E), "o": (E, H * D), "gate": (F, E), "up": (F, E),
            "down": (E, F)}
    types = [{"q": 2, "k": 10, "v": 11, "o": 1, "gate": 12, "up": 14, "down": 2},
             {"q": 0, "k": 11, "v": 10, "o": 2, "gate": 14, "up": 12, "down": 1}]
    base_layers, head = LM.make(cfg, 0, seed=34)
    layers = []
    for l in range(cfg["n_layers"]):
        lw = {"attn_norm": base_layers[l]["attn_norm"], "ffn_norm": base_layers[l]["ffn_norm"]}
        for m in LM.MATS:
            lw[m] = _tensor(*rows[m], types[l][m], 100 * l + len(m))
        layers.append(lw)
    head = {"out_norm": head["out_norm"], "lm": _tensor(V, E, 0, 77)}
    embd = (_tensor(V, E, 10, 78), 10)
    ids = {}
    for l in range(cfg["n_layers"]):
        for m in LM.MATS:
            ids[(l, m)] = 1000 + 10 * l + LM.MATS.index(m)
            GM.GTYPE[ids[(l, m)]] = types[l][m]
    GM.GTYPE[999] = 0
    path = str(tmp_path / "reference_loader.gguf")
    try:
        GM.write_model(path, cfg, layers, head, embd, 2,
                       [{m: ids[(l, m)] for m in LM.MATS} for l in range(cfg["n_layers"])], 999)
    finally:
        for k in list(GM.GTYPE):
            if k >= 999:
                del GM.GTYPE[k]
    m = llama.DecodeModel.from_gguf(path, dev, max_seq=cfg["max_seq"])
    assert m.plan["loader"] == "reference"
    q8 = []
    for l in range(cfg["n_layers"]):
        q8l = {"attn_norm": layers[l]["attn_norm"], "ffn_norm": layers[l]["ffn_norm"]}
        for name in LM.MATS:
            n, k = rows[name]
            want = O.q8_pad64(O.dequant_py(layers[l][name], types[l][name]).reshape(n, k), n, k)
            got = to_np(m.keep[3 + l][name])
            assert np.array_equal(got, want), f"layer {l} {name} padded weights"
            q8l[name] = _pad64_to_q8_0_rows(want, n, k)
        q8.append(q8l)
    lm_pad = O.q8_pad64(O.dequant_py(head["lm"], 0).reshape(V, E), V, E)
    assert np.array_equal(to_np(m.lm_head), lm_pad), "head padded weights"
    lm_rows = _pad64_to_q8_0_rows(lm_pad, V, E)
    table = O.dequant_py(embd[0], 10).reshape(V, E)
    ko, vo = LM.caches(cfg)
    for pos, tok_in in enumerate([5, 17, 299]):
        print(f"reference loader position {pos}", flush=True)
        emb = m.embed(tok_in)
        assert_bits_equal(to_np(emb), table[tok_in], "embedding row")
        want = O.ref_llama_step(q8, cfg, ko, vo, pos, table[tok_in], head["out_norm"], lm_rows, V)
        if want is None:
            pytest.skip("oracle/_ref not built")
        tok = m.step(emb, pos)
        assert tok == want[0], f"token at {pos}"
        assert_bits_equal(to_np(m.buf_t["logits"]), want[3], f"logits at {pos}")
