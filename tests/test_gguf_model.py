"""The GGUF model assembler's host side (bpd_substrate_amd.llama.gguf_plan):
metadata -> config, blk.N.* tensors -> per-matrix formats and byte ranges,
the head (output.weight, or token_embd when tied), rope_dim and
rope_freqs.weight, and the errors for files the decode step cannot run.
The reference reads the same keys and names (inference/llamatov_c_inference.py:
114-182)."""
import numpy as np
import pytest

import gguf_model as GM
import llama_model as LM
from bpd_substrate_amd import gguf, llama

Q4KM = {"v": 4, "down": 4}


def _model(tmp_path, name="m.gguf", **kw):
    cfg = LM.config(L=2, vocab=300)
    fm = [dict(Q4KM), {}]
    layers, head = LM.make(cfg, 2, seed=31, formats=fm, lm_fmt=4)
    embd = (LM.synth.q4k(cfg["vocab_size"], cfg["n_embd"], LM.synth.key(31, 5)), gguf.Q4_K)
    args = dict(rope_dim=32, rope_freqs=np.linspace(1, 4, 16).astype(np.float32))
    args.update(kw)
    path = str(tmp_path / name)
    GM.write_model(path, cfg, layers, head, embd, 2, fm, 4, **args)
    return path, cfg, layers, head, embd


def test_plan_of_a_q4k_m_file(tmp_path):
    path, cfg, layers, head, embd = _model(tmp_path)
    g = gguf.open_gguf(path)
    plan = llama.gguf_plan(g, max_seq=64)
    got = dict(plan["cfg"])
    assert np.float32(got.pop("eps")) == np.float32(cfg["eps"])   # stored as F32
    assert got == {k: v for k, v in cfg.items() if k != "eps"}
    assert plan["rope_dim"] == 32 and plan["rope_freqs"].name == "rope_freqs.weight"
    for l, lw in enumerate(plan["layers"]):
        for m in LM.MATS:
            t, f = lw[m]
            want = (Q4KM if l == 0 else {}).get(m, llama.W_Q4K_GGUF)
            assert f == want, (l, m)
            assert bytes(g.tensor_bytes(t.name)) == layers[l][m].tobytes()
        assert lw["q_bias"] is None
    t, f = plan["head"]
    assert t.name == "output.weight" and f == llama.W_Q6K_GGUF
    assert bytes(g.tensor_bytes(t.name)) == head["lm"].tobytes()
    assert bytes(g.tensor_bytes(plan["embd"].name)) == embd[0].tobytes()


def test_plan_tied_head_and_defaults(tmp_path):
    path, cfg, *_ = _model(tmp_path, tied=True, rope_dim=None, rope_freqs=None)
    plan = llama.gguf_plan(gguf.open_gguf(path))
    assert plan["head"][0].name == "token_embd.weight" and plan["head"][1] == llama.W_Q4K_GGUF
    assert plan["rope_dim"] == cfg["head_dim"] and plan["rope_freqs"] is None
    assert plan["cfg"]["max_seq"] == 2048


@pytest.mark.parametrize("bad", ["missing", "dims", "mix", "f16_matrix", "freqs", "q5k_matrix"])
def test_plan_rejects(tmp_path, bad):
    cfg = LM.config(L=1, vocab=300)
    layers, head = LM.make(cfg, 2, seed=32, lm_fmt=2)
    embd = (LM.synth.q4k(cfg["vocab_size"], cfg["n_embd"], LM.synth.key(32, 5)), gguf.Q4_K)
    path = str(tmp_path / "bad.gguf")
    if bad == "missing":
        GM.write_model(path, cfg, layers, head, embd, 2, None, 2)
        g = gguf.open_gguf(path)
        del g.by_name["blk.0.ffn_up.weight"]
        with pytest.raises(gguf.GGUFError, match="blk.0.ffn_up.weight is missing"):
            llama.gguf_plan(g)
        return
    if bad == "dims":
        GM.write_model(path, cfg, layers, head, embd, 2, None, 2)
        g = gguf.open_gguf(path)
        g.metadata["llama.attention.head_count_kv"] = 1      # K and V would be 64 rows, the file holds 128
        with pytest.raises(gguf.GGUFError, match="attn_k.weight has dims"):
            llama.gguf_plan(g)
        return
    if bad == "mix":
        layers[0]["o"] = LM.synth.q8_0(cfg["n_embd"], cfg["n_embd"], LM.synth.key(32, 9))
        GM.write_model(path, cfg, layers, head, embd, 2, [{"o": 0}], 2)
        match = "cannot be combined"
    elif bad in ("f16_matrix", "q5k_matrix"):
        f16 = bad == "f16_matrix"
        n = cfg["ff_dim"] * cfg["n_embd"]
        layers[0]["up"] = np.zeros(n, np.float16) if f16 else np.zeros(n // 256 * 176, np.uint8)
        GM.GTYPE[99] = 1 if f16 else 13
        try:
            GM.write_model(path, cfg, layers, head, embd, 2, [{"up": 99}], 2)
        finally:
            del GM.GTYPE[99]
        match = "not a decode-step weight format"
    else:
        GM.write_model(path, cfg, layers, head, embd, 2, None, 2, rope_dim=32, rope_freqs=np.ones(8, np.float32))
        match = "rope_freqs.weight has dims"
    g = gguf.open_gguf(path)
    with pytest.raises(gguf.GGUFError, match=match):
        llama.gguf_plan(g, loader="native")
    if bad in ("mix", "f16_matrix"):
        # the reference loader reads both (every matrix dequantized and re-quantized to
        # the padded Q8 layout), and "auto" falls back to it
        plan = llama.gguf_plan(g)
        assert plan["loader"] == "reference" and plan["head"][1] == llama.W_Q8_PAD64
        assert {f for lw in plan["layers"] for m, _ in llama._GGUF_MATS for f in [lw[m][1]]} == {llama.W_Q8_PAD64}
    elif bad == "q5k_matrix":  # no loader reads Q5_K: "auto" reports the native loader's error
        with pytest.raises(gguf.GGUFError, match="no loader formula"):
            llama.gguf_plan(g, loader="reference")
        with pytest.raises(gguf.GGUFError, match=match):
            llama.gguf_plan(g)
    else:
        with pytest.raises(gguf.GGUFError, match=match):
            llama.gguf_plan(g)
