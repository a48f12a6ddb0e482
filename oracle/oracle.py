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
LIB = os.path.join(HERE, "liboracle.so")
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


def qmatmul_q8_0_llamafile(W, X, m_weight, m_tokens, K, order="T"):
    out = np.empty(m_weight * m_tokens, np.float32)
    lib().bpdq_o_qmatmul_q8_0_llamafile(_p(W), _p(X), _p(out), m_weight, m_tokens, K, ord(order))
    return out


def dequant_q4k_mt(q, nthreads):
    nb = q.size // 144
    out = np.empty(nb * 256, np.float32)
    lib().bpdq_o_dequant_q4k_mt(_p(q), _p(out), nb, nthreads)
    return out
