"""Small random llama-shaped models for the decode-step tests (numpy, host).

Weights are seeded synthetic tensors (bpd_substrate_amd.synth): Q8_0 rows
[N][K/32][34] (fmt 0) or Q4_K rows [N][K/256][144] (fmt 1, 2); norm weights
N(1, 0.1); biases N(0, 0.1).  `to_device` builds the GPU copy in the layout the
library takes (the padded Q8 layout for fmt 0)."""
import numpy as np

from bpd_substrate_amd import formats, synth

MATS = ("q", "k", "v", "o", "gate", "up", "down")


def config(E=256, H=4, HKV=2, D=64, F=512, L=2, vocab=1000, max_seq=64, eps=1e-5, theta=10000.0):
    return dict(n_layers=L, n_embd=E, n_head=H, n_head_kv=HKV, head_dim=D, ff_dim=F, vocab_size=vocab,
                max_seq=max_seq, eps=eps, rope_theta=theta)


def _norm_w(n, k):
    return (1.0 + 0.1 * synth.normal_f32(n, k)).astype(np.float32)


def q6k(n, k, key, d_sigma=0.0001):
    """Q6_K rows [n][k/256][210]: random quant and scale bytes, f16 d ~ |N(0, d_sigma)|."""
    nb = n * (k // 256)
    b = synth.random_bytes(nb * 210, key).reshape(nb, 210)
    b[:, 208:210] = (np.abs(synth.normal_f32(nb, key ^ 0x5A5A)) * d_sigma).astype(np.float16).view(np.uint8) \
        .reshape(nb, 2)
    return b.reshape(-1)


def make(cfg, fmt=0, seed=1, bias=False, f32_head=False, formats=None, lm_fmt=None):
    """formats: per layer, {matrix: format} for matrices not in `fmt` (3/4: Q6_K)."""
    E, H, HKV, D, F = (cfg[n] for n in ("n_embd", "n_head", "n_head_kv", "head_dim", "ff_dim"))
    shapes = {"q": (H * D, E), "k": (HKV * D, E), "v": (HKV * D, E), "o": (E, H * D),
              "gate": (F, E), "up": (F, E), "down": (E, F)}
    s = 1000 * seed

    def mat(n, k, key, f=fmt):
        if f == 0:
            return synth.q8_0(n, k, key, d_sigma=0.002)
        if f in (3, 4):
            return q6k(n, k, key)
        return synth.q4k(n, k, key, d_sigma=0.0005, dmin_sigma=0.0003)

    layers = []
    for l in range(cfg["n_layers"]):
        lw = {"attn_norm": _norm_w(E, synth.key(s + l, 1)), "ffn_norm": _norm_w(E, synth.key(s + l, 2))}
        for i, m in enumerate(MATS):
            lw[m] = mat(*shapes[m], synth.key(s + l, 10 + i), (formats[l] if formats else {}).get(m, fmt))
        if bias:
            lw["q_bias"] = 0.1 * synth.normal_f32(H * D, synth.key(s + l, 30))
            lw["k_bias"] = 0.1 * synth.normal_f32(HKV * D, synth.key(s + l, 31))
            lw["v_bias"] = 0.1 * synth.normal_f32(HKV * D, synth.key(s + l, 32))
        layers.append(lw)
    vocab = cfg["vocab_size"]
    head = {"out_norm": _norm_w(E, synth.key(s + 99, 1))}
    if f32_head:
        head["lm"] = None
        head["lm_f32"] = (0.05 * synth.normal_f32(vocab * E, synth.key(s + 99, 2))).astype(np.float32)
    else:
        head["lm"] = mat(vocab, E, synth.key(s + 99, 3), fmt if lm_fmt is None else lm_fmt)
        head["lm_f32"] = None
    return layers, head


def embeddings(cfg, n, seed=7):
    return [synth.normal_f32(cfg["n_embd"], synth.key(seed, 100 + i)) for i in range(n)]


def to_device(cfg, layers, head, fmt, dev):
    """(device layer dicts, out_norm, lm_head, lm_f32) as torch tensors."""
    import torch

    E, H, D, F = cfg["n_embd"], cfg["n_head"], cfg["head_dim"], cfg["ff_dim"]
    rows = {"q": (H * D, E), "k": (cfg["n_head_kv"] * D, E), "v": (cfg["n_head_kv"] * D, E), "o": (E, H * D),
            "gate": (F, E), "up": (F, E), "down": (E, F)}

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    def w(a, n, k):
        return t(formats.q8_0_rows_to_pad64(a, n, k) if fmt == 0 else a)

    dl = []
    for lw in layers:
        d = {"attn_norm": t(lw["attn_norm"]), "ffn_norm": t(lw["ffn_norm"])}
        for m in MATS:
            d[m] = w(lw[m], *rows[m])
        for b in ("q_bias", "k_bias", "v_bias"):
            d[b] = t(lw[b]) if b in lw else None
        dl.append(d)
    lm = None if head["lm"] is None else w(head["lm"], cfg["vocab_size"], E)
    lm_f32 = None if head["lm_f32"] is None else t(head["lm_f32"])
    return dl, t(head["out_norm"]), lm, lm_f32


def caches(cfg, f16=False):
    n = cfg["max_seq"] * cfg["n_head_kv"] * cfg["head_dim"]
    dt = np.uint16 if f16 else np.float32
    return ([np.zeros(n, dt) for _ in range(cfg["n_layers"])],
            [np.zeros(n, dt) for _ in range(cfg["n_layers"])])
