"""Synthetic GGUF model files for the assembler tests: llama.cpp's tensor names
and {arch}.* metadata, with the numpy tensors of llama_model.make written as
GGUF bytes (dims ne[0] = row length first)."""
import numpy as np

import llama_model as LM
from bpd_substrate_amd import gguf

GNAMES = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
          "down": "ffn_down"}
GTYPE = {0: gguf.Q8_0, 1: gguf.Q4_K, 2: gguf.Q4_K, 3: gguf.Q6_K, 4: gguf.Q6_K}


def write_model(path, cfg, layers, head, embd, base, formats, lm_fmt, rope_dim=None, rope_freqs=None, tied=False,
                extra_meta=()):
    E, H, HKV, D, F, V = (cfg[n] for n in ("n_embd", "n_head", "n_head_kv", "head_dim", "ff_dim", "vocab_size"))
    rows = {"q": (H * D, E), "k": (HKV * D, E), "v": (HKV * D, E), "o": (E, H * D), "gate": (F, E), "up": (F, E),
            "down": (E, F)}
    md = [("general.architecture", gguf.T_STR, "llama"), ("general.quantization_version", gguf.T_U32, 3),
          ("llama.block_count", gguf.T_U32, cfg["n_layers"]), ("llama.embedding_length", gguf.T_U32, E),
          ("llama.feed_forward_length", gguf.T_U32, F), ("llama.attention.head_count", gguf.T_U32, H),
          ("llama.attention.head_count_kv", gguf.T_U32, HKV),
          ("llama.attention.layer_norm_rms_epsilon", gguf.T_F32, cfg["eps"]),
          ("llama.rope.freq_base", gguf.T_F32, cfg["rope_theta"]), ("llama.vocab_size", gguf.T_U32, V)]
    if rope_dim is not None:
        md.append(("llama.rope.dimension_count", gguf.T_U32, rope_dim))
    md += list(extra_meta)
    tensors = [("token_embd.weight", (E, V), embd[1], embd[0].tobytes())]
    if rope_freqs is not None:
        tensors.append(("rope_freqs.weight", (len(rope_freqs),), 0, np.asarray(rope_freqs, np.float32).tobytes()))
    for l, lw in enumerate(layers):
        p = f"blk.{l}"
        tensors.append((f"{p}.attn_norm.weight", (E,), 0, lw["attn_norm"].tobytes()))
        for m in LM.MATS:
            n, k = rows[m]
            f = (formats[l] if formats else {}).get(m, base)
            tensors.append((f"{p}.{GNAMES[m]}.weight", (k, n), GTYPE[f], lw[m].tobytes()))
        tensors.append((f"{p}.ffn_norm.weight", (E,), 0, lw["ffn_norm"].tobytes()))
    tensors.append(("output_norm.weight", (E,), 0, head["out_norm"].tobytes()))
    if not tied:
        tensors.append(("output.weight", (E, V), GTYPE[lm_fmt], head["lm"].tobytes()))
    gguf.write_gguf(path, md, tensors)
