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

W_Q8_PAD64, W_Q4K, W_Q4K_GGUF, W_Q6K, W_Q6K_GGUF = 0, 1, 2, 3, 4


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


class StepOpts(ctypes.Structure):    # include/bpdq_llama.h bpd_llama_step_opts
    _fields_ = [
        ("layer_formats", ctypes.POINTER(ctypes.c_int)), ("lm_format", ctypes.c_int),
        ("rope_dim", ctypes.c_int), ("rope_freqs", ctypes.POINTER(ctypes.c_float)),
        ("kv_cache_f16", ctypes.c_int),
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
    The extended step (bpd_llama_step_ext_gpu) is used when any of these is given:
    formats: per layer, a dict {matrix name: W_*} for matrices not in `fmt`
         (a Q4_K_M file keeps attn_v and ffn_down in Q6_K);
    lm_format: the head's format (default `fmt`);
    rope_dim, rope_freqs (numpy float32 [rope_dim/2], kept on the host);
    kv_cache_f16: binary16 caches (torch.int16 tensors holding the bits).
    """

    def __init__(self, cfg, layers, out_norm, lm_head=None, lm_f32=None, lm_N=None, fmt=W_Q8_PAD64, device=None,
                 formats=None, lm_format=None, rope_dim=None, rope_freqs=None, kv_cache_f16=False):
        import numpy as np
        import torch

        self.fmt = fmt
        self.ext = (formats is not None or lm_format is not None or rope_dim is not None or rope_freqs is not None
                    or kv_cache_f16)
        nl = max(1, cfg["n_layers"])
        fm = [[(formats[l] if formats else {}).get(m, fmt) for m in MATRICES] for l in range(cfg["n_layers"])]
        self._fmts = (ctypes.c_int * (7 * nl))(*[f for row in fm for f in row])
        self._freqs = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
        self.opts = StepOpts(ctypes.cast(self._fmts, ctypes.POINTER(ctypes.c_int)) if formats else None,
                             -1 if lm_format is None else lm_format, rope_dim or 0,
                             None if self._freqs is None else self._freqs.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                             1 if kv_cache_f16 else 0)
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
        cdt = torch.int16 if kv_cache_f16 else torch.float32
        self.k_cache = [z(S * HKV * D, cdt) for _ in range(L)]
        self.v_cache = [z(S * HKV * D, cdt) for _ in range(L)]
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
        if self.fmt == W_Q8_PAD64 and not self.ext:
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
        if self.ext:
            rc = gpu.call("bpd_llama_step_ext_gpu", self.fmt, ctypes.addressof(self.opts), *self._args(emb, pos))
        else:
            rc = gpu.call("bpd_llama_step_gpu", self.fmt, *self._args(emb, pos))
        if rc != 0:
            gpu.check()


# ---- the reference's CPU transformer ABI (bench/bpd_cpu.c:5556-5604), on the GPU ----
# Field for field the ctypes structs of the reference's CPU driver
# (bench/bpd_llamatov_infer.py:45-83), so its build_model() output binds unchanged.
_fp = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class BpdLlamaConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int), ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int), ("embed_dim", ctypes.c_int), ("ffn_dim", ctypes.c_int),
        ("vocab_size", ctypes.c_int), ("max_seq_len", ctypes.c_int),
        ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float),
        ("rope_dim", ctypes.c_int), ("kv_cache_f16", ctypes.c_int),
    ]


class BpdLlamaLayerWeights(ctypes.Structure):
    _fields_ = [
        ("attn_norm_w", _fp), ("w_q", _u8p), ("w_k", _u8p), ("w_v", _u8p), ("w_o", _u8p),
        ("ffn_norm_w", _fp), ("w_gate", _u8p), ("w_up", _u8p), ("w_down", _u8p),
    ]


class BpdLlamaWeights(ctypes.Structure):
    _fields_ = [
        ("token_embd", _u8p), ("layers", ctypes.POINTER(BpdLlamaLayerWeights)),
        ("output_norm_w", _fp), ("output_w", _u8p), ("rope_freqs", _fp),
    ]


_REF_LAYER = ("attn_norm_w", "w_q", "w_k", "w_v", "w_o", "ffn_norm_w", "w_gate", "w_up", "w_down")


def layer_struct(lw):
    """BpdLlamaLayerWeights of device tensors keyed by the struct's field names."""
    s = BpdLlamaLayerWeights()
    for n, t in BpdLlamaLayerWeights._fields_:
        setattr(s, n, ctypes.cast(lw[n].data_ptr(), t))
    return s


class Forward:
    """A model in the reference CPU ABI's layout on the device: Q8_0 weights
    (GGUF bytes), fp32 norms, caches of n_layers * max_seq_len rows in
    binary16 (torch.int16 bits) or fp32.  forward() is bpd_llama_forward_gpu
    (or the _s_ form with order="S"):

        f = Forward(cfg, layers, token_embd, output_norm, output_w, rope_freqs=None)
        logits, tokens = f.forward(token_ids, pos_ids, kv_pos)

    cfg: dict with BpdLlamaConfig's field names; layers: dicts of device tensors
    with BpdLlamaLayerWeights' field names."""

    def __init__(self, cfg, layers, token_embd, output_norm, output_w, rope_freqs=None, device=None):
        import numpy as np
        import torch

        self.cfg = BpdLlamaConfig(*(cfg[n] for n, _ in BpdLlamaConfig._fields_))
        L, S, HKV, D = cfg["n_layers"], cfg["max_seq_len"], cfg["n_kv_heads"], cfg["head_dim"]
        dev = device if device is not None else output_norm.device
        self.keep = [layers, token_embd, output_norm, output_w]
        self.layers = (BpdLlamaLayerWeights * max(1, L))(*[layer_struct(lw) for lw in layers])
        self._freqs = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
        self.w = BpdLlamaWeights(ctypes.cast(token_embd.data_ptr(), _u8p),
                                 ctypes.cast(self.layers, ctypes.POINTER(BpdLlamaLayerWeights)),
                                 ctypes.cast(output_norm.data_ptr(), _fp), ctypes.cast(output_w.data_ptr(), _u8p),
                                 None if self._freqs is None else self._freqs.ctypes.data_as(_fp))
        cdt = torch.int16 if cfg["kv_cache_f16"] else torch.float32
        self.k_cache = torch.zeros(max(1, L) * S * HKV * D, dtype=cdt, device=dev)
        self.v_cache = torch.zeros(max(1, L) * S * HKV * D, dtype=cdt, device=dev)
        self.device = dev

    def forward(self, token_ids, pos_ids, kv_pos, order="T"):
        """Returns device tensors (logits [n][vocab_size] fp32, tokens [n] int64)."""
        import numpy as np
        import torch

        ids = np.ascontiguousarray(token_ids, np.int32)
        pos = np.ascontiguousarray(pos_ids, np.int32)
        n = ids.size
        logits = torch.empty(max(1, n) * self.cfg.vocab_size, dtype=torch.float32, device=self.device)
        toks = torch.empty(max(1, n), dtype=torch.int64, device=self.device)
        gpu._use_torch_stream()
        gpu.call("bpd_llama_forward_s_gpu" if order == "S" else "bpd_llama_forward_gpu", ids.ctypes.data, n,
                 ctypes.addressof(self.w), ctypes.addressof(self.cfg), pos.ctypes.data, int(kv_pos), self.k_cache,
                 self.v_cache, logits, toks)
        return logits[: n * self.cfg.vocab_size], toks[:n]


# ---- a decode model straight from a GGUF file ----
# The reference driver's loader (inference/llamatov_c_inference.py:114-182) reads
# the {arch}.* metadata into ModelConfig and every blk.N.* tensor into
# LayerWeights, dequantizing each tensor type on the host
# (inference/llamatov_helpers.py:195-222) and re-quantizing to the padded Q8
# layout.  Two loaders here:
# * native: the bytes go to the device unchanged and each matrix keeps its own
#   format: Q4_K and Q6_K run as themselves (GGUF element map), an all-Q8_0 model
#   takes the padded Q8 layout;
# * reference: the reference driver's weights, for every type its loader reads
#   (F32, F16, Q4_0, Q2_K, Q3_K, Q4_K, Q6_K): each matrix and the head dequantized
#   on the device with load_tensor_by_type's formulas (bpd_dequant_gguf_py_gpu),
#   then re-quantized to the padded Q8 layout (bpd_q8_pad64_from_f32_gpu, the
#   reference's q8_pad64_coalesced), and the token table kept in fp32.
#   load_tensor_by_type has no Q8_0 branch (it returns zeros for it); Q8_0
#   tensors take the reference C's Q8_0 dequant (bpd_dequant_q8_0_gpu) instead.
# loader="auto" takes the native one when every matrix is Q4_K, Q6_K or Q8_0 in
# a combination the step runs, else the reference one.

# the GGUF types the reference loader reads (load_tensor_by_type), and Q8_0
PY_TYPES = (0, 1, 2, 10, 11, 12, 14)


def load_tensor_by_type(path, offset, n_elements, shape, type_code, device):
    """inference/llamatov_helpers.py:196-222 with the dequant on `device`: the tensor of
    `n_elements` at byte `offset` of the file as an fp32 device tensor of `shape`.  An
    unknown type gives zeros and a warning, as the reference's does."""
    import numpy as np
    import torch

    if type_code not in PY_TYPES:
        print(f"  WARN: unknown type code {type_code}, using zeros")
        return torch.zeros(shape, dtype=torch.float32, device=device)
    per, size = gpu.GGUF_PY_BLOCKS[type_code]
    raw = np.fromfile(path, dtype=np.uint8, count=n_elements // per * size, offset=offset)
    out = gpu.dequant_gguf_py(torch.from_numpy(raw).to(device), n_elements, type_code)
    return out.reshape(shape)

_GGUF_MATS = (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
              ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down"))


def _gguf_format(t, loader="native"):
    from . import gguf

    if loader == "reference":
        if t.type in PY_TYPES or t.type == gguf.Q8_0:
            return W_Q8_PAD64
        raise gguf.GGUFError(f"{t.name}: type {t.type_name} has no loader formula "
                             "(F32, F16, Q4_0, Q2_K, Q3_K, Q4_K, Q6_K, Q8_0)")
    if t.type == gguf.Q4_K:
        return W_Q4K_GGUF
    if t.type == gguf.Q6_K:
        return W_Q6K_GGUF
    if t.type == gguf.Q8_0:
        return W_Q8_PAD64
    raise gguf.GGUFError(f"{t.name}: type {t.type_name} is not a decode-step weight format (Q4_K, Q6_K, Q8_0); "
                         "loader='reference' reads it")


def gguf_plan(g, max_seq=2048, loader="auto"):
    """Host-side reading of a parsed GGUF (gguf.GGUF) as a decode model: returns
    dict(cfg, layers=[{matrix: (tensor, format), norms, biases}], head=(tensor, format or
    None for fp32), embd=tensor, out_norm=tensor, rope_dim, rope_freqs=tensor or None,
    loader="native" or "reference").  Raises gguf.GGUFError for a missing tensor, a shape
    that does not match the metadata, or formats the loader cannot take."""
    from . import gguf

    if loader not in ("auto", "native", "reference"):
        raise ValueError(f"loader {loader!r}: 'auto', 'native' or 'reference'")
    if loader == "auto":
        try:
            return gguf_plan(g, max_seq, "native")
        except gguf.GGUFError as e:
            try:
                return gguf_plan(g, max_seq, "reference")
            except gguf.GGUFError:
                raise e from None

    md = g.metadata
    arch = md.get("general.architecture", "llama")

    def meta(key, default=None):
        v = md.get(f"{arch}.{key}", default)
        if v is None:
            raise gguf.GGUFError(f"metadata {arch}.{key} is missing")
        return v

    def need(name, dims=None):
        if name not in g.by_name:
            raise gguf.GGUFError(f"tensor {name} is missing")
        t = g.by_name[name]
        if dims is not None and tuple(t.dims) != tuple(dims):
            raise gguf.GGUFError(f"tensor {name} has dims {t.dims}, expected {tuple(dims)}")
        return t

    L, E, H = int(meta("block_count")), int(meta("embedding_length")), int(meta("attention.head_count"))
    HKV = int(md.get(f"{arch}.attention.head_count_kv", H))
    if H <= 0 or E % H:
        raise gguf.GGUFError(f"embedding_length {E} is not a multiple of head_count {H}")
    D = E // H
    F = int(need("blk.0.ffn_gate.weight").dims[1]) if L > 0 else int(md.get(f"{arch}.feed_forward_length", 0))
    head_t = g.by_name.get("output.weight") or need("token_embd.weight")
    V = int(md.get(f"{arch}.vocab_size", head_t.dims[1]))
    cfg = dict(n_layers=L, n_embd=E, n_head=H, n_head_kv=HKV, head_dim=D, ff_dim=F, vocab_size=V, max_seq=max_seq,
               eps=float(md.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-5)),
               rope_theta=float(md.get(f"{arch}.rope.freq_base", 500000.0)))
    rope_dim = int(md.get(f"{arch}.rope.dimension_count", D))
    rdims = {"q": (E, H * D), "k": (E, HKV * D), "v": (E, HKV * D), "o": (H * D, E), "gate": (E, F), "up": (E, F),
             "down": (F, E)}
    layers = []
    for l in range(L):
        p = f"blk.{l}"
        lw = {"attn_norm": need(f"{p}.attn_norm.weight", (E,)), "ffn_norm": need(f"{p}.ffn_norm.weight", (E,))}
        for m, gname in _GGUF_MATS:
            t = need(f"{p}.{gname}.weight", rdims[m])
            lw[m] = (t, _gguf_format(t, loader))
        for b, gname, n in (("q_bias", "attn_q", H * D), ("k_bias", "attn_k", HKV * D), ("v_bias", "attn_v", HKV * D)):
            key = f"{p}.{gname}.bias"
            lw[b] = need(key, (n,)) if key in g.by_name else None
        layers.append(lw)
    need(head_t.name, (E, V))
    if loader == "reference":  # the reference's head: output.weight or token_embd, in the padded layout
        head_fmt = _gguf_format(head_t, loader)
        emb_t = need("token_embd.weight", (E, V))
        if emb_t.type not in PY_TYPES and emb_t.type != gguf.Q8_0:
            raise gguf.GGUFError(f"token_embd.weight: type {emb_t.type_name} has no loader formula")
    else:
        head_fmt = None if head_t.type in (0, 1) else _gguf_format(head_t)
    fmts = {f for lw in layers for m, _ in _GGUF_MATS for f in [lw[m][1]]} | ({head_fmt} - {None})
    if W_Q8_PAD64 in fmts and len(fmts) > 1:
        raise gguf.GGUFError("Q8_0 matrices cannot be combined with K-quant ones in one decode step")
    rf = g.by_name.get("rope_freqs.weight")
    if rf is not None and tuple(rf.dims) != (rope_dim // 2,):
        raise gguf.GGUFError(f"rope_freqs.weight has dims {rf.dims}, expected ({rope_dim // 2},)")
    return dict(cfg=cfg, layers=layers, head=(head_t, head_fmt), embd=need("token_embd.weight", (E, V)),
                out_norm=need("output_norm.weight", (E,)), rope_dim=rope_dim, rope_freqs=rf, loader=loader)


def _f32_tensor(g, t, device):
    import numpy as np
    import torch

    raw = np.frombuffer(g.tensor_bytes(t.name), np.uint8)
    if t.type == 0:
        a = raw.view(np.float32)
    elif t.type == 1:
        a = raw.view(np.float16).astype(np.float32)
    else:
        raise ValueError(f"{t.name}: expected F32 or F16, found {t.type_name}")
    return torch.from_numpy(a.copy()).to(device)


def _f32_of(g, t, device):
    """fp32 of a GGUF tensor on the device as the reference loader computes it
    (Q8_0: the reference C's dequant)."""
    from . import gguf

    raw = g.to_device(t.name, device)
    n = t.n_elements
    if t.type == gguf.Q8_0:
        return gpu.dequant_q8_0(raw)
    return gpu.dequant_gguf_py(raw, n, t.type)


def from_gguf(path, device, max_seq=2048, kv_cache_f16=False, loader="auto"):
    """A DecodeModel of the GGUF file at `path` (see gguf_plan and the loaders above),
    with .embed(token_id) -> the token's fp32 embedding row on the device."""
    import numpy as np

    from . import formats as fm
    from . import gguf

    g = gguf.open_gguf(path)
    plan = gguf_plan(g, max_seq, loader)
    cfg = plan["cfg"]
    E = cfg["n_embd"]
    ref = plan["loader"] == "reference"

    def weight(t, f):
        if ref:  # fp32, then the reference's q8_pad64_coalesced, rows = dims[1]
            return gpu.q8_pad64(_f32_of(g, t, device), t.dims[1], t.dims[0])
        if f != W_Q8_PAD64:
            return g.to_device(t.name, device)
        import torch   # Q8_0 rows -> the padded layout of the padded-Q8 step

        host = np.frombuffer(g.tensor_bytes(t.name), np.uint8)
        return torch.from_numpy(fm.q8_0_rows_to_pad64(host, t.dims[1], t.dims[0])).to(device)

    layers, formats = [], []
    for lw in plan["layers"]:
        d = {"attn_norm": _f32_tensor(g, lw["attn_norm"], device), "ffn_norm": _f32_tensor(g, lw["ffn_norm"], device)}
        for m, _ in _GGUF_MATS:
            d[m] = weight(*lw[m])
        for b in ("q_bias", "k_bias", "v_bias"):
            d[b] = None if lw[b] is None else _f32_tensor(g, lw[b], device)
        layers.append(d)
        formats.append({m: lw[m][1] for m, _ in _GGUF_MATS})
    head_t, head_fmt = plan["head"]
    base = formats[0]["q"] if formats else (head_fmt if head_fmt is not None else W_Q4K_GGUF)
    lm = None if head_fmt is None else weight(head_t, head_fmt)
    lm_f32 = _f32_tensor(g, head_t, device) if head_fmt is None else None
    freqs = None
    if plan["rope_freqs"] is not None:
        freqs = np.frombuffer(g.tensor_bytes(plan["rope_freqs"].name), np.uint8).view(np.float32).copy()
    # the reference loader's model is all padded Q8: the reference's own generate_token
    # ABI unless RoPE options or binary16 caches need the extended step
    m = DecodeModel(cfg, layers, _f32_tensor(g, plan["out_norm"], device), lm_head=lm, lm_f32=lm_f32,
                    lm_N=head_t.dims[1], fmt=base, device=device, formats=None if ref else formats,
                    lm_format=None if ref else (head_fmt if head_fmt is not None else base),
                    rope_dim=None if ref and plan["rope_dim"] == cfg["head_dim"] else plan["rope_dim"],
                    rope_freqs=freqs, kv_cache_f16=kv_cache_f16)
    m.gguf, m.plan = g, plan
    m._embd = g.to_device(plan["embd"].name, device)
    m._embd_f32 = _f32_of(g, plan["embd"], device) if ref else None
    return m


def _embed(self, token):
    """The fp32 embedding row of `token` on the device, as the GPU entry points compute
    it: the Q8_0 lookup, or the GGUF-map dequant of the row's Q4_K / Q6_K blocks."""
    import torch

    from . import gguf

    t = self.plan["embd"]
    E = self.cfg.n_embd
    if not 0 <= token < t.dims[1]:
        raise ValueError(f"token {token} outside 0..{t.dims[1] - 1}")
    gpu._use_torch_stream()
    out = torch.empty(E, dtype=torch.float32, device=self._embd.device)
    if getattr(self, "_embd_f32", None) is not None:  # the reference loader's fp32 table
        out.copy_(self._embd_f32[token * E:(token + 1) * E])
    elif t.type == gguf.Q8_0:
        ids = torch.tensor([token], dtype=torch.int32, device=self._embd.device)
        gpu.call("bpd_embed_lookup_q8_0_gpu", self._embd, ids, out, 1, E)
    elif t.type in (gguf.Q4_K, gguf.Q6_K):
        bpb = 144 if t.type == gguf.Q4_K else 210
        nb = E // 256
        row = self._embd[token * nb * bpb:(token + 1) * nb * bpb]   # 16-byte (Q4_K) / 2-byte (Q6_K) aligned
        gpu.call("bpd_dequant_q4k_gguf_gpu" if t.type == gguf.Q4_K else "bpd_dequant_q6k_gguf_gpu", row, out, nb)
    elif t.type == 0:
        out.copy_(self._embd.view(torch.float32)[token * E:(token + 1) * E])
    else:
        raise ValueError(f"token_embd type {t.type_name} has no embedding lookup")
    return out


DecodeModel.from_gguf = staticmethod(from_gguf)
DecodeModel.embed = _embed
