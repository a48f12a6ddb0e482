"""The GEMV chain of one llama decode step over Q4_K weights, on the GPU.

Per layer this issues the seven weight GEMVs of the reference's block
(bench/bpd_cpu.c:5642-5733: Q, K, V, O, gate, up, down) as Q4_K x Q8_K GEMVs,
each activation quantized to Q8_K first:

    xa = Q8_K(attn_in)   ->  q, k, v = Wq xa, Wk xa, Wv xa      (one fused launch)
    xo = Q8_K(attn_out)  ->  o = Wo xo
    xf = Q8_K(ffn_in)    ->  g, u = Wgate xf, Wup xf            (one fused launch)
    xh = Q8_K(ffn_mid)   ->  d = Wdown xh

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

    def __init__(self, layers, dims=Dims(), device=None):
        import torch

        self.L = load_hip()
        self.layers = layers
        self.d = dims
        dev = device or layers[0].q.device
        e, kv, ff = dims.n_embd, dims.n_kv, dims.ff
        q8k = lambda n: torch.empty(n // formats.Q8K_ELEMS * formats.Q8K_BYTES, dtype=torch.uint8, device=dev)
        self.xa, self.xo, self.xf, self.xh = q8k(e), q8k(e), q8k(e), q8k(ff)
        f32 = lambda n: torch.empty(n, dtype=torch.float32, device=dev)
        self.out = [dict(q=f32(e), k=f32(kv), v=f32(kv), o=f32(e), gate=f32(ff), up=f32(ff), down=f32(e))
                    for _ in layers]

    def _multi(self, ws, ys, Ms, xq, K):
        n = len(ws)
        w_arr = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
        y_arr = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        m_arr = (ctypes.c_int * n)(*Ms)
        self.L.bpd_qmatmul_q4k_q8k_multi_gpu(w_arr, y_arr, m_arr, n, xq.data_ptr(), K)

    def layer(self, i, attn_in, attn_out, ffn_in, ffn_mid):
        """Launch layer i's chain (asynchronous, on the library's current stream)."""
        L, d, w, o = self.L, self.d, self.layers[i], self.out[i]
        e, kv, ff = d.n_embd, d.n_kv, d.ff
        L.bpd_quant_q8_k_gpu(attn_in.data_ptr(), self.xa.data_ptr(), e)
        self._multi([w.q, w.k, w.v], [o["q"], o["k"], o["v"]], [e, kv, kv], self.xa, e)
        L.bpd_quant_q8_k_gpu(attn_out.data_ptr(), self.xo.data_ptr(), e)
        L.bpd_qmatmul_q4k_q8k_gpu(w.o.data_ptr(), self.xo.data_ptr(), o["o"].data_ptr(), e, e)
        L.bpd_quant_q8_k_gpu(ffn_in.data_ptr(), self.xf.data_ptr(), e)
        self._multi([w.gate, w.up], [o["gate"], o["up"]], [ff, ff], self.xf, e)
        L.bpd_quant_q8_k_gpu(ffn_mid.data_ptr(), self.xh.data_ptr(), ff)
        L.bpd_qmatmul_q4k_q8k_gpu(w.down.data_ptr(), self.xh.data_ptr(), o["down"].data_ptr(), e, ff)

    def step(self, acts):
        """One token: every layer's chain; acts[i] = (attn_in, attn_out, ffn_in, ffn_mid)."""
        for i in range(len(self.layers)):
            self.layer(i, *acts[i])

    def weight_bytes(self):
        d = self.d
        per = formats.q4k_bytes(d.n_embd, d.n_embd) * 2 + formats.q4k_bytes(d.n_kv, d.n_embd) * 2 \
            + formats.q4k_bytes(d.ff, d.n_embd) * 2 + formats.q4k_bytes(d.n_embd, d.ff)
        return per * len(self.layers)
