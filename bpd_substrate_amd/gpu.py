"""Host-side mirror of the reference's GPU entry points, over libbpdq_hip.so.

Two layers:

* `call(name, *args)` — the C ABI exactly as the reference's ctypes callers
  use it (bench/verify_quant_gpu.py:27-42 and friends): device pointers as ints,
  sizes as ints.  Torch tensors are accepted wherever a pointer is and are
  passed as their data_ptr().  After the call the library's error slot is read
  and a BpdqError is raised if the arguments were rejected or HIP failed.
* tensor helpers (`dequant_q4k`, `qmatmul_q4k_q8k`, ...) that allocate the
  outputs as torch tensors on the current device and launch on torch's current
  stream.

Nothing here computes on the CPU: if libbpdq_hip.so is not built, every entry
point raises.
"""
import ctypes

from . import formats
from ._native import load_hip


class BpdqError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"bpdq error {code}: {msg}")
        self.code = code


def lib():
    return load_hip()


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    if isinstance(a, ctypes.c_void_p):
        return a.value
    raise TypeError(f"cannot pass {type(a).__name__} as a device pointer")


def check():
    """Raise BpdqError if the last call on this thread recorded an error."""
    L = lib()
    code = L.bpd_gpu_last_error()
    if code:
        raise BpdqError(code, L.bpd_gpu_last_error_message().decode())


def call(name, *args):
    """Call an exported entry point by name; pointers may be tensors.  Only names with a
    declared ctypes signature are callable: without one, ctypes would pass each Python
    int as a 32-bit C int and cut 64-bit device pointers short."""
    from ._native import HIP_SIGNATURES

    if name not in HIP_SIGNATURES:
        raise KeyError(f"{name} has no ctypes signature in _native.HIP_SIGNATURES")
    fn = getattr(lib(), name)
    conv = [_ptr(a) if not isinstance(a, (float,)) else a for a in args]
    res = fn(*conv)
    check()
    return res


BPDQ_ERR_SHAPE = 2  # include/bpdq.h


def _need(t, nbytes, what):
    """The C ABI takes bare device pointers and cannot see buffer sizes, so the tensor
    helpers check them here: t must be contiguous and hold at least nbytes."""
    if t is None or isinstance(t, int) or not hasattr(t, "numel"):
        return
    if not t.is_contiguous():
        raise BpdqError(BPDQ_ERR_SHAPE, f"{what} is not contiguous")
    have = t.numel() * t.element_size()
    if have < nbytes:
        raise BpdqError(BPDQ_ERR_SHAPE, f"{what} holds {have} bytes, the call needs {nbytes}")


def _q4k_bytes(M, K):
    return max(M, 0) * max(K, 0) // 256 * formats.Q4K_BYTES


def _q8k_bytes(K):
    return max(K, 0) // formats.Q8K_ELEMS * formats.Q8K_BYTES


def _q8_0_bytes(rows, K):
    return max(rows, 0) * max(K, 0) // 32 * formats.Q8_0_BYTES


def _use_torch_stream():
    import torch

    lib().bpd_gpu_set_stream(torch.cuda.current_stream().cuda_stream)


def _empty(n, dtype, like):
    import torch

    return torch.empty(n, dtype=dtype, device=like.device)


# ---------------------------------------------------------------- Q4_K / Q8_K

def dequant_q4k(q, order=formats.ORDER_BPD, out=None):
    """q: uint8 device tensor of n_blocks*144 bytes -> fp32 tensor [n_blocks*256]."""
    import torch

    nb = q.numel() // formats.Q4K_BYTES
    out = _empty(nb * 256, torch.float32, q) if out is None else out
    _need(out, nb * 256 * 4, "out")
    _use_torch_stream()
    call("bpd_dequant_q4k_gpu" if order == formats.ORDER_BPD else "bpd_dequant_q4k_gguf_gpu", q, out, nb)
    return out


def qmatmul_q4k(w, x, M, K, out=None):
    """Reference-order GEMV, fp32 x (bit-identical to bpd_qmatmul_q4k)."""
    import torch

    out = _empty(M, torch.float32, x) if out is None else out
    _need(w, _q4k_bytes(M, K), "w")
    _need(x, max(K, 0) * 4, "x")
    _need(out, max(M, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q4k_gpu", w, x, out, M, K)
    return out


def quant_q8_k(x, out=None):
    import torch

    n = x.numel()
    out = _empty(n // formats.Q8K_ELEMS * formats.Q8K_BYTES, torch.uint8, x) if out is None else out
    _need(out, _q8k_bytes(n), "out")
    _use_torch_stream()
    call("bpd_quant_q8_k_gpu", x, out, n)
    return out


def qmatmul_q4k_q8k(w, xq, M, K, order=formats.ORDER_BPD, out=None):
    import torch

    out = _empty(M, torch.float32, xq) if out is None else out
    _need(w, _q4k_bytes(M, K), "w")
    _need(xq, _q8k_bytes(K), "xq")
    _need(out, max(M, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q4k_q8k_gpu" if order == formats.ORDER_BPD else "bpd_qmatmul_q4k_q8k_gguf_gpu",
         w, xq, out, M, K)
    return out


def qmatmul_q4k_q8k_multi(ws, xq, Ms, K, outs=None):
    """Up to four Q4_K GEMVs sharing the activation xq, in one launch."""
    return _multi("bpd_qmatmul_q4k_q8k_multi_gpu", ws, xq, Ms, K, outs)


def qmatmul_q4k_q8k_fused(w, x, M, K, out=None):
    """Q4_K x Q8_K(x) for fp32 x, quantized inside the GEMV kernel (bits equal quant + GEMV)."""
    import torch

    out = _empty(M, torch.float32, x) if out is None else out
    _need(w, _q4k_bytes(M, K), "w")
    _need(x, max(K, 0) * 4, "x")
    _need(out, max(M, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q4k_q8k_fused_gpu", w, x, out, M, K)
    return out


def qmatmul_q4k_q8k_fused_multi(ws, x, Ms, K, outs=None):
    """Up to four Q4_K GEMVs of one fp32 activation, quantized in-kernel, in one launch."""
    return _multi("bpd_qmatmul_q4k_q8k_fused_multi_gpu", ws, x, Ms, K, outs)


def _multi(name, ws, x, Ms, K, outs):
    import torch

    n = len(ws)
    outs = [_empty(m, torch.float32, x) for m in Ms] if outs is None else outs
    for i in range(n):
        _need(ws[i], _q4k_bytes(Ms[i], K), f"w[{i}]")
        _need(outs[i], max(Ms[i], 0) * 4, f"out[{i}]")
    _need(x, max(K, 0) * 4 if "fused" in name else _q8k_bytes(K), "x")
    w_arr = (ctypes.c_void_p * n)(*[_ptr(w) for w in ws])
    y_arr = (ctypes.c_void_p * n)(*[_ptr(y) for y in outs])
    m_arr = (ctypes.c_int * n)(*Ms)
    _use_torch_stream()
    call(name, ctypes.addressof(w_arr), ctypes.addressof(y_arr), ctypes.addressof(m_arr), n, x, K)
    return outs


# ---------------------------------------------------------------- padded Q8 layout

def q8_pad64(x, N, K, out=None):
    """fp32 [N, K] -> uint8 [K/32 * N * 64] in the layout of q8_pad64_coalesced
    (inference/llamatov_c_inference.py:88-100)."""
    import torch

    out = _empty(K // 32 * N * 64, torch.uint8, x) if out is None else out
    _need(x, max(N, 0) * max(K, 0) * 4, "x")
    _need(out, max(K, 0) // 32 * max(N, 0) * 64, "out")
    _use_torch_stream()
    call("bpd_q8_pad64_from_f32_gpu", x, out, N, K)
    return out


def qmatmul_q8_pad64(Wp, Xq, m_weight, m_tokens, K, out=None):
    import torch

    out = _empty(m_tokens * m_weight, torch.float32, Xq) if out is None else out
    _need(Wp, max(K, 0) // 32 * max(m_weight, 0) * 64, "W_pad64")
    _need(Xq, _q8_0_bytes(m_tokens, K), "Xq")
    _need(out, max(m_tokens * m_weight, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q8_pad64_gpu", Wp, Xq, out, m_weight, m_tokens, K)
    return out


# ---------------------------------------------------------------- the reference Python loader

# elements and bytes per block of the types load_tensor_by_type dequantizes
# (inference/llamatov_helpers.py:196-222)
GGUF_PY_BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 10: (256, 84), 11: (256, 110), 12: (256, 144), 14: (256, 210)}


def dequant_gguf_py(raw, n_elements, ggml_type, out=None):
    """raw: uint8 device tensor of a GGUF tensor's bytes -> fp32 [n_elements] with the
    reference Python loader's formula for ggml_type (bpd_dequant_gguf_py_gpu)."""
    import torch

    if ggml_type not in GGUF_PY_BLOCKS:
        raise ValueError(f"ggml_type {ggml_type} has no loader formula")
    per, size = GGUF_PY_BLOCKS[ggml_type]
    out = _empty(n_elements, torch.float32, raw) if out is None else out
    _need(raw, n_elements // per * size, "raw")
    _need(out, n_elements * 4, "out")
    _use_torch_stream()
    call("bpd_dequant_gguf_py_gpu", raw, out, n_elements, ggml_type)
    return out


# ---------------------------------------------------------------- Q6_K

def dequant_q6k(q, order=formats.ORDER_BPD, out=None):
    """q: uint8 device tensor of n_blocks*210 bytes -> fp32 [n_blocks*256].  ORDER_BPD is the
    reference's map (inference/llamatov_helpers.py:161-179), ORDER_GGUF llama.cpp's."""
    import torch

    nb = q.numel() // 210
    out = _empty(nb * 256, torch.float32, q) if out is None else out
    _need(out, nb * 256 * 4, "out")
    _use_torch_stream()
    call("bpd_dequant_q6k_gpu" if order == formats.ORDER_BPD else "bpd_dequant_q6k_gguf_gpu", q, out, nb)
    return out


def qmatmul_q6k_q8k(w, xq, M, K, order=formats.ORDER_BPD, out=None):
    import torch

    out = _empty(M, torch.float32, xq) if out is None else out
    _need(w, max(M, 0) * max(K, 0) // 256 * 210, "w")
    _need(xq, _q8k_bytes(K), "xq")
    _need(out, max(M, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q6k_q8k_gpu" if order == formats.ORDER_BPD else "bpd_qmatmul_q6k_q8k_gguf_gpu",
         w, xq, out, M, K)
    return out


# ---------------------------------------------------------------- Q8_0

def dequant_q8_0(raw, out=None):
    import torch

    nb = raw.numel() // formats.Q8_0_BYTES
    out = _empty(nb * 32, torch.float32, raw) if out is None else out
    _need(out, nb * 32 * 4, "out")
    _use_torch_stream()
    call("bpd_dequant_q8_0_gpu", raw, out, nb)
    return out


def embed_lookup_q8_0(table, ids, embed_dim, out=None):
    import torch

    n = ids.numel()
    out = _empty(n * embed_dim, torch.float32, table) if out is None else out
    _need(table, _q8_0_bytes(1, embed_dim), "table")   # ids index rows on the device: 0 <= id < rows
    _need(out, n * max(embed_dim, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_embed_lookup_q8_0_gpu", table, ids, out, n, embed_dim)
    return out


def quant_q8_0(x, out=None):
    import torch

    n = x.numel()
    out = _empty(n // 32 * 34, torch.uint8, x) if out is None else out
    _need(out, n // 32 * 34, "out")
    _use_torch_stream()
    call("bpd_quant_q8_0_gpu", x, out, n)
    return out


def qmatmul_q8_0_dispatch(Wq, Xq, m_weight, m_tokens, K, out=None):
    """out[token * m_weight + row] in the AVX1 llamafile tile order."""
    import torch

    out = _empty(m_tokens * m_weight, torch.float32, Wq) if out is None else out
    _need(Wq, _q8_0_bytes(m_weight, K), "Wq")
    _need(Xq, _q8_0_bytes(m_tokens, K), "Xq")
    _need(out, max(m_tokens * m_weight, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q8_0_dispatch_gpu", Wq, Xq, out, m_weight, m_tokens, K)
    return out


def qmatmul_q8_0_llamafile(W, X, m_weight, m_tokens, K, out=None):
    import torch

    out = _empty(m_tokens * m_weight, torch.float32, W) if out is None else out
    _need(W, _q8_0_bytes(m_weight, K), "W")
    _need(X, max(m_tokens, 0) * max(K, 0) * 4, "X")
    _need(out, max(m_tokens * m_weight, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q8_0_llamafile_gpu", W, X, out, m_weight, m_tokens, K)
    return out


def qmatmul_q8_0_dispatch_s(Wq, Xq, m_weight, m_tokens, K, out=None):
    """out[token * m_weight + row] in the scalar order S (int8 MFMA prefill GEMM)."""
    import torch

    out = _empty(m_tokens * m_weight, torch.float32, Wq) if out is None else out
    _need(Wq, _q8_0_bytes(m_weight, K), "Wq")
    _need(Xq, _q8_0_bytes(m_tokens, K), "Xq")
    _need(out, max(m_tokens * m_weight, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q8_0_dispatch_s_gpu", Wq, Xq, out, m_weight, m_tokens, K)
    return out


def qmatmul_q8_0_llamafile_s(W, X, m_weight, m_tokens, K, out=None):
    import torch

    out = _empty(m_tokens * m_weight, torch.float32, W) if out is None else out
    _need(W, _q8_0_bytes(m_weight, K), "W")
    _need(X, max(m_tokens, 0) * max(K, 0) * 4, "X")
    _need(out, max(m_tokens * m_weight, 0) * 4, "out")
    _use_torch_stream()
    call("bpd_qmatmul_q8_0_llamafile_s_gpu", W, X, out, m_weight, m_tokens, K)
    return out
