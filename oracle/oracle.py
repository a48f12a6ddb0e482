"""ctypes binding of the C oracle (liboracle.so) and of the reference C built
from source into oracle/_ref/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# BPDQ_ORACLE_LIB: another build of the same file (the sanitized one, make san)
LIB = os.environ.get("BPDQ_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_LIBS = {
    "quant": os.path.join(REF_DIR, "bpd_quant_ref.so"),        # bench/bpd_quant.c, -O2
    "scalar": os.path.join(REF_DIR, "bpd_cpu_scalar_ref.so"),  # bpd_cpu.c + bpd_gemm_q8_0_cpu.c, -O2
    "avx": os.path.join(REF_DIR, "bpd_cpu_avx_ref.so"),        # same, -O2 -mavx -mssse3
}

P, I, F, U16 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_uint16

_SIGS = {
    "bpdq_o_f16_ldexp": (F, [U16]),
    "bpdq_o_f16_magic": (F, [U16]),
    "bpdq_o_f16_h2h": (F, [U16]),
    "bpdq_o_f32_to_f16": (U16, [F]),
    "bpdq_o_dequant_q4k": (None, [P, P, I]),
    "bpdq_o_dequant_q4k_gguf": (None, [P, P, I]),
    "bpdq_o_qmatmul_q4k": (None, [P, P, P, I, I]),
    "bpdq_o_qmm_q4k": (None, [P, P, P, I, I, I]),
    "bpdq_o_quant_q8_k": (None, [P, P, I]),
    "bpdq_o_qmatmul_q4k_q8k": (None, [P, P, P, I, I, I]),
    "bpdq_o_q4k_q8k_block_ints": (None, [P, P, I, P, P]),
    "bpdq_o_q8_pad64": (None, [P, P, I, I]),
    "bpdq_o_q6k_quants": (None, [P, I, P]),
    "bpdq_o_dequant_q6k": (None, [P, P, I, I]),
    "bpdq_o_q6k_q8k_block_int": (ctypes.c_int32, [P, P, I]),
    "bpdq_o_qmatmul_q6k_q8k": (None, [P, P, P, I, I, I]),
    "bpdq_o_qmatmul_q6k_q8k_mt": (None, [P, P, P, I, I, I, I]),
    "bpdq_o_dequant_q8_0": (None, [P, P, I]),
    "bpdq_o_embed_lookup_q8_0": (None, [P, P, P, I, I]),
    "bpdq_o_quant_q8_0": (None, [P, P, I]),
    "bpdq_o_qdot_q8_0_S": (F, [P, P, I]),
    "bpdq_o_qdot_q8_0_P": (F, [P, P, I]),
    "bpdq_o_cell_q8_0_T": (F, [P, P, I]),
    "bpdq_o_cell_q8_0_S": (F, [P, P, I]),
    "bpdq_o_dispatch_q8_0": (None, [P, P, P, I, I, I, I]),
    "bpdq_o_qmatmul_q8_0": (None, [P, P, P, I, I, I, I]),
    "bpdq_o_qmatmul_q8_0_llamafile": (None, [P, P, P, I, I, I, I]),
    "bpdq_o_dequant_q4k_mt": (None, [P, P, I, I]),
    "bpdq_o_qmatmul_q4k_q8k_mt": (None, [P, P, P, I, I, I, I]),
    "bpdq_o_dispatch_q8_0_mt": (None, [P, P, P, I, I, I, I, I]),
    "bpdq_o_expf_nagy": (F, [F]),
    "bpdq_o_expf_table": (None, [P]),
    "bpdq_o_expf_mismatches": (ctypes.c_uint64, [I, ctypes.c_uint32, P]),
    "bpdq_o_libm_expf": (None, [P, P, I]),
    "bpdq_o_rmsnorm": (None, [P, P, P, I, F]),
    "bpdq_o_rope_norm": (None, [P, I, I, I, F]),
    "bpdq_o_gqa_attn": (None, [P, P, P, P, I, I, I, I, I, F]),
    "bpdq_o_swiglu": (None, [P, P, P, I]),
    "bpdq_o_argmax": (I, [P, I]),
    "bpdq_o_gemv_f32_wave": (None, [P, P, P, I, I]),
    "bpdq_o_llama_step": (I, [I, P, P, P, P, I, P, P, P, P, I, P, P, P]),
    "bpdq_o_llama_step_ext": (I, [P, P, P, P, P, I, P, P, P, P, I, P, P, P]),
    "bpdq_o_rope_norm_freqs": (None, [P, I, I, I, F, I, P]),
    "bpdq_o_f16_numpy": (F, [ctypes.c_uint16]),
    "bpdq_o_dequant_f16": (None, [P, P, ctypes.c_int64]),
    "bpdq_o_dequant_q4_0": (None, [P, P, I]),
    "bpdq_o_dequant_q2k_py": (None, [P, P, I]),
    "bpdq_o_dequant_q3k_py": (None, [P, P, I]),
    "bpdq_o_dequant_q4k_py": (None, [P, P, I]),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def ref(kind):
    """The reference C library of the given build, or None if it is not built."""
    path = REF_LIBS[kind]
    return ctypes.CDLL(path) if os.path.exists(path) else None


def _p(a):
    return a.ctypes.data


# ------------------------------------------------------------------ wrappers

def dequant_q4k(q):
    nb = q.size // 144
    out = np.empty(nb * 256, np.float32)
    lib().bpdq_o_dequant_q4k(_p(q), _p(out), nb)
    return out


def dequant_q4k_gguf(q):
    nb = q.size // 144
    out = np.empty(nb * 256, np.float32)
    lib().bpdq_o_dequant_q4k_gguf(_p(q), _p(out), nb)
    return out


def qmatmul_q4k(w, x, M, K):
    y = np.empty(M, np.float32)
    lib().bpdq_o_qmatmul_q4k(_p(w), _p(x), _p(y), M, K)
    return y


def qmm_q4k(A, B, M, N, K):
    C = np.empty(M * N, np.float32)
    lib().bpdq_o_qmm_q4k(_p(A), _p(B), _p(C), M, N, K)
    return C


def quant_q8_k(x):
    y = np.empty(x.size // 256 * 292, np.uint8)
    lib().bpdq_o_quant_q8_k(_p(x), _p(y), x.size)
    return y


def qmatmul_q4k_q8k(w, xq, M, K, order=0, nthreads=1):
    y = np.empty(M, np.float32)
    if nthreads > 1:
        lib().bpdq_o_qmatmul_q4k_q8k_mt(_p(w), _p(xq), _p(y), M, K, order, nthreads)
    else:
        lib().bpdq_o_qmatmul_q4k_q8k(_p(w), _p(xq), _p(y), M, K, order)
    return y


def block_ints(wblk, xblk, order=0):
    I_, M_ = ctypes.c_int32(), ctypes.c_int32()
    lib().bpdq_o_q4k_q8k_block_ints(_p(wblk), _p(xblk), order, ctypes.addressof(I_), ctypes.addressof(M_))
    return I_.value, M_.value


def q8_pad64(x, N, K):
    out = np.empty(K // 32 * N * 64, np.uint8)
    lib().bpdq_o_q8_pad64(_p(np.ascontiguousarray(x, np.float32)), _p(out), N, K)
    return out


def q6k_quants(blk, order=0):
    q = np.empty(256, np.int8)
    lib().bpdq_o_q6k_quants(_p(blk), order, _p(q))
    return q


def dequant_q6k(q, order=0):
    nb = q.size // 210
    out = np.empty(nb * 256, np.float32)
    lib().bpdq_o_dequant_q6k(_p(q), _p(out), nb, order)
    return out


# the reference Python loader's per-type dequant (inference/llamatov_helpers.py:196-222)
PY_BLOCKS = {1: (1, 2), 2: (32, 18), 10: (256, 84), 11: (256, 110), 12: (256, 144), 14: (256, 210)}


def dequant_py(raw, ggml_type):
    """fp32 of a GGUF tensor's bytes as load_tensor_by_type computes it (F32, F16, Q4_0,
    Q2_K, Q3_K, Q4_K, Q6_K)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if ggml_type == 0:
        return raw.view(np.float32).copy()
    per, size = PY_BLOCKS[ggml_type]
    nb = raw.size // size
    out = np.empty(nb * per, np.float32)
    if ggml_type == 1:
        lib().bpdq_o_dequant_f16(_p(raw), _p(out), nb)
    elif ggml_type == 14:
        lib().bpdq_o_dequant_q6k(_p(raw), _p(out), nb, 0)
    else:
        fn = {2: "bpdq_o_dequant_q4_0", 10: "bpdq_o_dequant_q2k_py", 11: "bpdq_o_dequant_q3k_py",
              12: "bpdq_o_dequant_q4k_py"}[ggml_type]
        getattr(lib(), fn)(_p(raw), _p(out), nb)
    return out


def q6k_block_int(wblk, xblk, order=0):
    return int(lib().bpdq_o_q6k_q8k_block_int(_p(wblk), _p(xblk), order))


def qmatmul_q6k_q8k(w, xq, M, K, order=0, nthreads=1):
    y = np.empty(M, np.float32)
    if nthreads > 1:
        lib().bpdq_o_qmatmul_q6k_q8k_mt(_p(w), _p(xq), _p(y), M, K, order, nthreads)
    else:
        lib().bpdq_o_qmatmul_q6k_q8k(_p(w), _p(xq), _p(y), M, K, order)
    return y


def dequant_q8_0(raw):
    nb = raw.size // 34
    out = np.empty(nb * 32, np.float32)
    lib().bpdq_o_dequant_q8_0(_p(raw), _p(out), nb)
    return out


def embed_lookup_q8_0(table, ids, embed_dim):
    out = np.empty(ids.size * embed_dim, np.float32)
    lib().bpdq_o_embed_lookup_q8_0(_p(table), _p(ids), _p(out), ids.size, embed_dim)
    return out


def quant_q8_0(x):
    y = np.empty(x.size // 32 * 34, np.uint8)
    lib().bpdq_o_quant_q8_0(_p(x), _p(y), x.size)
    return y


def dispatch_q8_0(Wq, Xq, m_weight, m_tokens, K, order="T", nthreads=1):
    out = np.empty(m_weight * m_tokens, np.float32)
    if nthreads > 1:
        lib().bpdq_o_dispatch_q8_0_mt(_p(Wq), _p(Xq), _p(out), m_weight, m_tokens, K, ord(order), nthreads)
    else:
        lib().bpdq_o_dispatch_q8_0(_p(Wq), _p(Xq), _p(out), m_weight, m_tokens, K, ord(order))
    return out


def qmatmul_q8_0(W, X, M, N, K, order="P"):
    out = np.empty(M * N, np.float32)
    lib().bpdq_o_qmatmul_q8_0(_p(W), _p(X), _p(out), M, N, K, ord(order))
    return out


def qdot_grid(Wq, Xq, M, N, K, order="P"):
    """out[m * N + n] = bpdq_o_qdot_q8_0_{P,S}(Wq row n, Xq row m, K/32)."""
    nb = K // 32
    bpr = nb * 34
    f = lib().bpdq_o_qdot_q8_0_P if order == "P" else lib().bpdq_o_qdot_q8_0_S
    w0, x0 = Wq.ctypes.data, Xq.ctypes.data
    return np.array([f(w0 + n * bpr, x0 + m * bpr, nb) for m in range(M) for n in range(N)], np.float32)


def qmatmul_q8_0_llamafile(W, X, m_weight, m_tokens, K, order="T"):
    out = np.empty(m_weight * m_tokens, np.float32)
    lib().bpdq_o_qmatmul_q8_0_llamafile(_p(W), _p(X), _p(out), m_weight, m_tokens, K, ord(order))
    return out


def dequant_q4k_mt(q, nthreads):
    nb = q.size // 144
    out = np.empty(nb * 256, np.float32)
    lib().bpdq_o_dequant_q4k_mt(_p(q), _p(out), nb, nthreads)
    return out


# ------------------------------------------------------------------ the decode step

def expf_nagy(x):
    return np.float32(lib().bpdq_o_expf_nagy(float(np.float32(x))))


def expf_table():
    t = np.empty(32, np.uint64)
    lib().bpdq_o_expf_table(_p(t))
    return t


def expf_mismatches(nthreads=8, stride=1):
    """(count, first input bits) of non-NaN inputs k*stride where the restated
    expf and libm's differ."""
    first = ctypes.c_uint32()
    n = lib().bpdq_o_expf_mismatches(nthreads, stride, ctypes.addressof(first))
    return n, first.value


def libm_expf(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().bpdq_o_libm_expf(_p(x), _p(y), x.size)
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().bpdq_o_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), _p(y), x.size, eps)
    return y


def rope_norm(t, n_heads, head_dim, pos, base):
    t = np.array(t, np.float32)
    lib().bpdq_o_rope_norm(_p(t), n_heads, head_dim, pos, base)
    return t


def gqa_attn(q, kc, vc, max_seq, pos, H, HKV, D, scale):
    out = np.empty(H * D, np.float32)
    lib().bpdq_o_gqa_attn(_p(q), _p(kc), _p(vc), _p(out), max_seq, pos, H, HKV, D, scale)
    return out


def swiglu(g, u):
    y = np.empty_like(g)
    lib().bpdq_o_swiglu(_p(g), _p(u), _p(y), g.size)
    return y


def argmax(x):
    return lib().bpdq_o_argmax(_p(np.ascontiguousarray(x, np.float32)), x.size)


def gemv_f32_wave(W, x, N, K):
    y = np.empty(N, np.float32)
    lib().bpdq_o_gemv_f32_wave(_p(W), _p(x), _p(y), N, K)
    return y


class _OLayer(ctypes.Structure):
    _fields_ = [(n, P) for n in ("attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up", "down",
                                 "q_bias", "k_bias", "v_bias")]


class _OCfg(ctypes.Structure):
    _fields_ = [(n, I) for n in ("n_layers", "n_embd", "n_head", "n_head_kv", "head_dim", "ff_dim", "max_seq")] + \
        [("eps", F), ("rope_theta", F)]


def _addr(a):
    return None if a is None else a.ctypes.data


def llama_step(fmt, layers, cfg, k_cache, v_cache, pos, emb, out_norm, lm, lm_f32, lm_N):
    """One decode step of the restatement (bpdq_o_llama_step).  layers: dicts of
    numpy arrays (Q8_0 rows for fmt 0, Q4_K for 1/2); k_cache, v_cache: lists
    of fp32 [max_seq * HKV * D] arrays, updated in place.
    Returns (token, x, h, logits)."""
    E = cfg["n_embd"]
    arr = (_OLayer * max(1, len(layers)))()
    for i, lw in enumerate(layers):
        for n, _ in _OLayer._fields_:
            setattr(arr[i], n, _addr(lw.get(n)))
    c = _OCfg(*(cfg[n] for n, _ in _OCfg._fields_))
    kp = (P * max(1, len(k_cache)))(*[_p(t) for t in k_cache])
    vp = (P * max(1, len(v_cache)))(*[_p(t) for t in v_cache])
    x, h, logits = np.empty(E, np.float32), np.empty(E, np.float32), np.empty(lm_N, np.float32)
    tok = lib().bpdq_o_llama_step(fmt, ctypes.addressof(arr), ctypes.addressof(c), kp, vp, pos, _p(emb),
                                  _p(out_norm), _addr(lm), _addr(lm_f32), lm_N, _p(x), _p(h), _p(logits))
    return tok, x, h, logits


class _OStepOpts(ctypes.Structure):
    _fields_ = [("fmts", P), ("lm_fmt", I), ("rope_dim", I), ("rope_freqs", P), ("kv_f16", I)]


def llama_step_ext(fmts, lm_fmt, layers, cfg, k_cache, v_cache, pos, emb, out_norm, lm, lm_f32, lm_N, rope_dim=None,
                   rope_freqs=None, kv_f16=False):
    """bpdq_o_llama_step_ext: fmts [n_layers][7] (q k v o gate up down), lm_fmt, rope_dim
    (default head_dim), rope_freqs, binary16 caches (uint16 arrays) with kv_f16.
    Returns (token, x, h, logits)."""
    E = cfg["n_embd"]
    arr = (_OLayer * max(1, len(layers)))()
    for i, lw in enumerate(layers):
        for n, _ in _OLayer._fields_:
            setattr(arr[i], n, _addr(lw.get(n)))
    c = _OCfg(*(cfg[n] for n, _ in _OCfg._fields_))
    f = np.ascontiguousarray(np.array(fmts, np.int32).reshape(-1) if len(layers) else np.zeros(7, np.int32))
    fr = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
    o = _OStepOpts(_p(f), lm_fmt, rope_dim or cfg["head_dim"], _addr(fr), 1 if kv_f16 else 0)
    kp = (P * max(1, len(k_cache)))(*[_p(t) for t in k_cache])
    vp = (P * max(1, len(v_cache)))(*[_p(t) for t in v_cache])
    x, h, logits = np.empty(E, np.float32), np.empty(E, np.float32), np.empty(lm_N, np.float32)
    tok = lib().bpdq_o_llama_step_ext(ctypes.addressof(o), ctypes.addressof(arr), ctypes.addressof(c), kp, vp, pos,
                                      _p(emb), _p(out_norm), _addr(lm), _addr(lm_f32), lm_N, _p(x), _p(h),
                                      _p(logits))
    return tok, x, h, logits


# The reference's own block, compiled from bench/bpd_cpu.c into oracle/_ref.
class RefLlamaConfig(ctypes.Structure):      # bench/bpd_cpu.c:5556-5570
    _fields_ = [(n, I) for n in ("n_layers", "n_heads", "n_kv_heads", "head_dim", "embed_dim", "ffn_dim",
                                 "vocab_size", "max_seq_len")] + \
        [("rms_eps", F), ("rope_base", F), ("rope_dim", I), ("kv_cache_f16", I)]


class RefLayerWeights(ctypes.Structure):     # bench/bpd_cpu.c:5585-5595
    _fields_ = [(n, P) for n in ("attn_norm_w", "w_q", "w_k", "w_v", "w_o", "ffn_norm_w", "w_gate", "w_up",
                                 "w_down")]


def ref_llama_step(layers, cfg, k_cache, v_cache, pos, emb, out_norm, lm, lm_N, kind="avx", rope_dim=None,
                   rope_freqs=None, kv_f16=False):
    """One token through the reference's bpd_llama_block_cpu per layer
    (bench/bpd_cpu.c:5611-5737), then the head of bpd_llama_forward_cpu
    (:5779-5792: bpd_rmsnorm_llama_cpu, bpd_qmatmul_q8_0_llamafile_cpu,
    bpd_argmax_dim_cpu), with an fp32 cache per layer.  (The forward itself
    steps its per-layer cache pointer in uint16_t units, :5771-5773, which
    overlaps fp32 layers; the composition here gives each layer its own.)
    Returns (token, x, h, logits), or None if oracle/_ref is not built."""
    R = ref(kind)
    if R is None:
        return None
    for name, args in (("bpd_llama_block_cpu", [P, P, P, P, I, I, P, P, P, P, P, P]),
                       ("bpd_rmsnorm_llama_cpu", [P, P, P, I, I, F]),
                       ("bpd_qmatmul_q8_0_llamafile_cpu", [P, P, P, I, I, I]),
                       ("bpd_argmax_dim_cpu", [P, P, I, I, I])):
        f = getattr(R, name)
        f.argtypes, f.restype = args, None
    E, H, HKV, D, F_ = (cfg[n] for n in ("n_embd", "n_head", "n_head_kv", "head_dim", "ff_dim"))
    c = RefLlamaConfig(cfg["n_layers"], H, HKV, D, E, F_, lm_N, cfg["max_seq"], cfg["eps"], cfg["rope_theta"],
                       rope_dim or D, 1 if kv_f16 else 0)
    fr = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
    x = np.array(emb, np.float32)
    big = max(E, F_, H * D)
    s1, s2, s3 = (np.zeros(big, np.float32) for _ in range(3))
    pos_ids = np.array([pos], np.int32)
    for l, lw in enumerate(layers):
        w = RefLayerWeights(*(_addr(lw[n]) for n in ("attn_norm", "q", "k", "v", "o", "ffn_norm", "gate", "up",
                                                     "down")))
        R.bpd_llama_block_cpu(_p(x), ctypes.addressof(w), ctypes.addressof(c), _p(pos_ids), 1, pos, _p(k_cache[l]),
                              _p(v_cache[l]), _p(s1), _p(s2), _p(s3), _addr(fr))
    h = np.empty(E, np.float32)
    R.bpd_rmsnorm_llama_cpu(_p(x), _p(out_norm), _p(h), 1, E, cfg["eps"])
    logits = np.empty(lm_N, np.float32)
    R.bpd_qmatmul_q8_0_llamafile_cpu(_p(lm), _p(h), _p(logits), lm_N, 1, E)
    tok = np.zeros(1, np.int64)
    R.bpd_argmax_dim_cpu(_p(logits), _p(tok), 1, lm_N, 1)
    return int(tok[0]), x, h, logits


def _ref_sigs(R):
    for name, args in (("bpd_llama_block_cpu", [P, P, P, P, I, I, P, P, P, P, P, P]),
                       ("bpd_llama_forward_cpu", [P, I, P, P, P, I, P, P, P, P])):
        f = getattr(R, name)
        f.argtypes, f.restype = args, None


class RefLlamaWeights(ctypes.Structure):     # bench/bpd_cpu.c:5598-5604
    _fields_ = [("token_embd", P), ("layers", P), ("output_norm_w", P), ("output_w", P), ("rope_freqs", P)]


_REF_LAYER = ("attn_norm_w", "w_q", "w_k", "w_v", "w_o", "ffn_norm_w", "w_gate", "w_up", "w_down")


def ref_block(layer, cfg, x, pos_ids, kv_pos, k_cache, v_cache, rope_freqs=None, kind="avx"):
    """The reference's own bpd_llama_block_cpu (bench/bpd_cpu.c:5608-5737) from
    oracle/_ref on host arrays: layer is a dict of numpy arrays keyed by
    bpd_llama_layer_weights' field names (Q8_0 rows, fp32 norms); cfg a dict keyed
    by bpd_llama_config's; x fp32 [n_tokens * embed_dim], k_cache / v_cache this
    layer's caches (uint16 bits when cfg["kv_cache_f16"], else fp32), all updated
    in place.  Returns False when oracle/_ref is not built."""
    R = ref(kind)
    if R is None:
        return False
    _ref_sigs(R)
    c = RefLlamaConfig(*(cfg[n] for n, _ in RefLlamaConfig._fields_))
    w = RefLayerWeights(*(_addr(layer[n]) for n in _REF_LAYER))
    T = len(pos_ids)
    big = T * max(cfg["embed_dim"], cfg["ffn_dim"])
    s1, s2, s3 = (np.zeros(big, np.float32) for _ in range(3))
    pos = np.ascontiguousarray(pos_ids, np.int32)
    fr = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
    R.bpd_llama_block_cpu(_p(x), ctypes.addressof(w), ctypes.addressof(c), _p(pos), T, kv_pos, _p(k_cache),
                          _p(v_cache), _p(s1), _p(s2), _p(s3), _addr(fr))
    return True


def ref_forward(weights, cfg, token_ids, pos_ids, kv_pos, k_cache, v_cache, kind="avx"):
    """The reference's own bpd_llama_forward_cpu (bench/bpd_cpu.c:5740-5798) from
    oracle/_ref: weights is a dict {token_embd, layers (list of layer dicts as for
    ref_block), output_norm_w, output_w, rope_freqs (or None)}; the caches hold
    n_layers layers and are updated in place.  Returns (logits [n][vocab], tokens
    int64 [n]), or None when oracle/_ref is not built."""
    R = ref(kind)
    if R is None:
        return None
    _ref_sigs(R)
    c = RefLlamaConfig(*(cfg[n] for n, _ in RefLlamaConfig._fields_))
    lws = (RefLayerWeights * max(1, len(weights["layers"])))(
        *[RefLayerWeights(*(_addr(lw[n]) for n in _REF_LAYER)) for lw in weights["layers"]])
    fr = weights.get("rope_freqs")
    fr = None if fr is None else np.ascontiguousarray(fr, np.float32)
    W = RefLlamaWeights(_addr(weights["token_embd"]), ctypes.addressof(lws), _addr(weights["output_norm_w"]),
                        _addr(weights["output_w"]), _addr(fr))
    ids = np.ascontiguousarray(token_ids, np.int32)
    pos = np.ascontiguousarray(pos_ids, np.int32)
    n = ids.size
    logits = np.zeros(n * cfg["vocab_size"], np.float32)
    toks = np.zeros(n, np.int64)
    R.bpd_llama_forward_cpu(_p(ids), n, ctypes.addressof(W), ctypes.addressof(c), _p(pos), kv_pos, _p(k_cache),
                            _p(v_cache), _p(logits), _p(toks))
    return logits.reshape(n, cfg["vocab_size"]), toks
