"""Host side of the decode step (include/bpdq_llama.h, llama.hip).

The four ctypes structs are the reference driver's own
(inference/llamatov_c_inference.py:15-60), field for field, so that driver's
code fills and passes them unchanged.  `DecodeModel` holds the device tensors
of one model (torch tensors on the GPU; torch is only the allocator), the
structs that point at them, the work buffers and the K/V cache, and runs one
step per token through the C ABI:

    m = DecodeModel(cfg, layers, out_norm, lm_head=..., fmt=W_Q8_PAD64, device=dev)
    tok = m.step(embedding_row, position)          # generate_token()

Field meaning used here and in the library: X_K is the input width of matrix X
(its reduction length) and X_N its number of output rows.
"""
import ctypes

from . import gpu

W_Q8_PAD64, W_Q4K, W_Q4K_GGUF = 0, 1, 2


class LayerWeights(ctypes.Structure):
    _fields_ = [
        ("attn_norm", ctypes.c_void_p),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
        ("ffn_norm", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("q_K", ctypes.c_int), ("q_N", ctypes.c_int),
        ("k_K", ctypes.c_int), ("k_N", ctypes.c_int),
        ("v_K", ctypes.c_int), ("v_N", ctypes.c_int),
        ("o_K", ctypes.c_int), ("o_N", ctypes.c_int),
        ("gate_K", ctypes.c_int), ("gate_N", ctypes.c_int),
        ("up_K", ctypes.c_int), ("up_N", ctypes.c_int),
        ("down_K", ctypes.c_int), ("down_N", ctypes.c_int),
        ("q_bias", ctypes.c_void_p), ("k_bias", ctypes.c_void_p), ("v_bias", ctypes.c_void_p),
    ]


class ModelConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int), ("n_embd", ctypes.c_int),
        ("n_head", ctypes.c_int), ("n_head_kv", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("ff_dim", ctypes.c_int),
        ("vocab_size", ctypes.c_int),
        ("max_seq", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
    ]


class KVCache(ctypes.Structure):
    _fields_ = [
        ("k_cache", ctypes.POINTER(ctypes.c_void_p)),
        ("v_cache", ctypes.POINTER(ctypes.c_void_p)),
    ]


class WorkBuffers(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p), ("h", ctypes.c_void_p),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p), ("attn_out", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("ffn", ctypes.c_void_p),
        ("logits", ctypes.c_void_p), ("argmax_result", ctypes.c_void_p),
    ]


MATRICES = ("q", "k", "v", "o", "gate", "up", "down")


class DecodeModel:
    """One model on the device, ready for decode steps.

    cfg: dict with n_layers, n_embd, n_head, n_head_kv, head_dim, ff_dim,
         vocab_size, max_seq, eps, rope_theta.
    layers: list of dicts with device tensors attn_norm, ffn_norm (fp32) and
         q, k, v, o, gate, up, down (uint8, in `fmt`), optional q_bias,
         k_bias, v_bias (fp32).
    lm_head: uint8 device tensor in `fmt`, or None with lm_f32 (fp32 [lm_N, n_embd]).
    """

    def __init__(self, cfg, layers, out_norm, lm_head=None, lm_f32=None, lm_N=None, fmt=W_Q8_PAD64, device=None):
        import torch

        self.fmt = fmt
        self.cfg_d = dict(cfg)
        E, H, HKV, D, F = (cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["head_dim"], cfg["ff_dim"])
        L, S = cfg["n_layers"], cfg["max_seq"]
        self.lm_N = int(lm_N if lm_N is not None else cfg["vocab_size"])
        self.cfg = ModelConfig(L, E, H, HKV, D, F, cfg["vocab_size"], S, cfg["eps"], cfg["rope_theta"])
        self.keep = [out_norm, lm_head, lm_f32]
        dims = {"q": (E, H * D), "k": (E, HKV * D), "v": (E, HKV * D), "o": (H * D, E),
                "gate": (E, F), "up": (E, F), "down": (F, E)}
        self.layers = (LayerWeights * max(1, L))()
        for i, lw in enumerate(layers):
            s = self.layers[i]
            s.attn_norm, s.ffn_norm = lw["attn_norm"].data_ptr(), lw["ffn_norm"].data_ptr()
            for name in MATRICES:
                setattr(s, name, lw[name].data_ptr())
                setattr(s, name + "_K", dims[name][0])
                setattr(s, name + "_N", dims[name][1])
            for b in ("q_bias", "k_bias", "v_bias"):
                setattr(s, b, lw[b].data_ptr() if lw.get(b) is not None else None)
            self.keep.append(lw)
        dev = device if device is not None else out_norm.device
        z = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt, device=dev)
        self.buf_t = {"x": z(E), "h": z(E), "q": z(H * D), "k": z(HKV * D), "v": z(HKV * D),
                      "attn_out": z(H * D), "gate": z(F), "up": z(F), "ffn": z(E),
                      "logits": z(self.lm_N), "argmax_result": z(4, torch.int32)}
        self.buf = WorkBuffers(**{k: v.data_ptr() for k, v in self.buf_t.items()})
        self.k_cache = [z(S * HKV * D) for _ in range(L)]
        self.v_cache = [z(S * HKV * D) for _ in range(L)]
        self._kp = (ctypes.c_void_p * max(1, L))(*[t.data_ptr() for t in self.k_cache])
        self._vp = (ctypes.c_void_p * max(1, L))(*[t.data_ptr() for t in self.v_cache])
        self.kv = KVCache(ctypes.cast(self._kp, ctypes.POINTER(ctypes.c_void_p)),
                          ctypes.cast(self._vp, ctypes.POINTER(ctypes.c_void_p)))
        self.out_norm, self.lm_head, self.lm_f32 = out_norm, lm_head, lm_f32

    def _args(self, emb, pos):
        p = lambda t: None if t is None else t.data_ptr()
        return (ctypes.addressof(self.layers), ctypes.addressof(self.cfg), ctypes.addressof(self.buf),
                ctypes.addressof(self.kv), int(pos), p(emb), p(self.out_norm), p(self.lm_head), p(self.lm_f32),
                self.cfg.n_embd, self.lm_N)

    def step(self, emb, pos):
        """One token through every layer; returns the argmax token (waits)."""
        gpu._use_torch_stream()
        if self.fmt == W_Q8_PAD64:
            tok = gpu.call("generate_token", *self._args(emb, pos))
            if tok < 0:
                gpu.check()
            return tok
        self.enqueue(emb, pos)
        import torch

        torch.cuda.current_stream().synchronize()
        return int(self.buf_t["argmax_result"][0].item())

    def enqueue(self, emb, pos):
        """The same step, launched on torch's current stream without waiting;
        the token is left in buf_t['argmax_result']."""
        gpu._use_torch_stream()
        rc = gpu.call("bpd_llama_step_gpu", self.fmt, *self._args(emb, pos))
        if rc != 0:
            gpu.check()
