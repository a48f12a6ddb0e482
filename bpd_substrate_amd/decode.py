"""The GEMV chain of one llama decode step over Q4_K weights, on the GPU.

Per layer this issues the seven weight GEMVs of the reference's block
(bench/bpd_cpu.c:5642-5733: Q, K, V, O, gate, up, down) as Q4_K x Q8_K GEMVs,
each activation quantized to Q8_K first:

    xa = Q8_K(attn_in)   ->  q, k, v = Wq xa, Wk xa, Wv xa      (one multi-matrix launch)
    xo = Q8_K(attn_out)  ->  o = Wo xo
    xf = Q8_K(ffn_in)    ->  g, u = Wgate xf, Wup xf            (one multi-matrix launch)
    xh = Q8_K(ffn_mid)   ->  d = Wdown xh

With fused=True (the default) each quantization happens inside the GEMV kernel
that consumes it (bpd_qmatmul_q4k_q8k_fused*_gpu): 4 launches per layer instead
of 8, same bits.

The norms, RoPE, attention and SwiGLU between them are not part of this path
(the activations are inputs), which makes this the GEMV portion a decode step
streams: 122,683,392 weight bytes per Mistral-7B-shaped layer.
Everything runs through the C ABI (libbpdq_hip.so); nothing computes on the CPU.
"""
import ctypes
from dataclasses import dataclass

from . import formats
from ._native import load_hip


@dataclass
class LayerWeights:
    """Device tensors (uint8, GGUF Q4_K bytes) of one layer."""

    q: object
    k: object
    v: object
    o: object
    gate: object
    up: object
    down: object


@dataclass
class Dims:
    n_embd: int = 4096      # rows of Q and O, K of Q/K/V/O/gate/up
    n_kv: int = 1024        # rows of K and V (8 KV heads x 128)
    ff: int = 14336         # rows of gate and up, K of down


class GemvChain:
    """Buffers and launch sequence for the decode-step GEMV chain."""

    def __init__(self, layers, dims=Dims(), device=None, fused=True):
        import torch

        self.L = load_hip()
        self.layers = layers
        self.d = dims
        self.fused = fused
        dev = device or layers[0].q.device
        e, kv, ff = dims.n_embd, dims.n_kv, dims.ff
        q8k = lambda n: torch.empty(n // formats.Q8K_ELEMS * formats.Q8K_BYTES, dtype=torch.uint8, device=dev)
        self.xa, self.xo, self.xf, self.xh = q8k(e), q8k(e), q8k(e), q8k(ff)
        f32 = lambda n: torch.empty(n, dtype=torch.float32, device=dev)
        self.out = [dict(q=f32(e), k=f32(kv), v=f32(kv), o=f32(e), gate=f32(ff), up=f32(ff), down=f32(e))
                    for _ in layers]

    def _gemv(self, ws, ys, Ms, x, xq, K):
        """GEMVs of the weights ws on the fp32 activation x (xq: its Q8_K buffer)."""
        L, n = self.L, len(ws)
        w_arr = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
        y_arr = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        m_arr = (ctypes.c_int * n)(*Ms)
        if self.fused:
            L.bpd_qmatmul_q4k_q8k_fused_multi_gpu(w_arr, y_arr, m_arr, n, x.data_ptr(), K)
        else:
            L.bpd_quant_q8_k_gpu(x.data_ptr(), xq.data_ptr(), K)
            L.bpd_qmatmul_q4k_q8k_multi_gpu(w_arr, y_arr, m_arr, n, xq.data_ptr(), K)

    def layer(self, i, attn_in, attn_out, ffn_in, ffn_mid):
        """Launch layer i's chain (asynchronous, on the library's current stream)."""
        d, w, o = self.d, self.layers[i], self.out[i]
        e, kv, ff = d.n_embd, d.n_kv, d.ff
        self._gemv([w.q, w.k, w.v], [o["q"], o["k"], o["v"]], [e, kv, kv], attn_in, self.xa, e)
        self._gemv([w.o], [o["o"]], [e], attn_out, self.xo, e)
        self._gemv([w.gate, w.up], [o["gate"], o["up"]], [ff, ff], ffn_in, self.xf, e)
        self._gemv([w.down], [o["down"]], [e], ffn_mid, self.xh, ff)

    def step(self, acts):
        """One token: every layer's chain; acts[i] = (attn_in, attn_out, ffn_in, ffn_mid)."""
        for i in range(len(self.layers)):
            self.layer(i, *acts[i])

    def weight_bytes(self):
        d = self.d
        per = formats.q4k_bytes(d.n_embd, d.n_embd) * 2 + formats.q4k_bytes(d.n_kv, d.n_embd) * 2 \
            + formats.q4k_bytes(d.ff, d.n_embd) * 2 + formats.q4k_bytes(d.n_embd, d.ff)
        return per * len(self.layers)
