"""CPU-only checks of the C ABI and the host code (no kernel is launched).

* libbpdq_hip.so loads and exports every function include/bpdq.h declares, and
  the Python signature table covers exactly that set.
* Argument validation rejects bad calls before any HIP call: error code set,
  message set, nothing launched.  (Each call below fails validation, so it
  runs safely without a GPU.)
* The synthetic generator is deterministic and chunking-invariant.
* bench.py refuses more than one GPU.
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from bpd_substrate_amd import _native, formats, synth
from bpd_substrate_amd import gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    inc = os.path.join(ROOT, "include")
    src = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", src, flags=re.M)
    return sorted(set(n for n in names if n not in ("defined",)))


def test_header_matches_exports_and_signatures():
    names = header_functions()
    assert len(names) >= 39
    lib = _native.load_hip()
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/bpdq.h but not exported"
    assert sorted(_native.HIP_SIGNATURES) == names


def test_exported_symbols_are_exactly_the_header(tmp_path):
    out = subprocess.run(["nm", "-D", "--defined-only", _native.HIP_LIB], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    ours = {n for n in exported if not n.startswith(("_", "__hip"))}
    assert set(header_functions()) <= ours


def _err(expected):
    L = _native.load_hip()
    code = L.bpd_gpu_last_error()
    msg = L.bpd_gpu_last_error_message().decode()
    assert code == expected, (code, msg)
    assert L.bpd_gpu_last_error() == 0  # cleared by the read
    return msg


def test_validation_rejects_before_launch():
    L = _native.load_hip()
    L.bpd_gpu_last_error()
    L.bpd_qmatmul_q4k_q8k_gpu(None, None, None, 4, 300)
    assert "multiple of 256" in _err(2)
    L.bpd_qmatmul_q4k_q8k_gpu(None, None, None, -1, 256)
    _err(2)
    L.bpd_qmatmul_q4k_q8k_gpu(0x1000, None, 0x2000, 4, 256)
    assert "NULL" in _err(1)
    L.bpd_qmatmul_q4k_q8k_gpu(0x1004, 0x2000, 0x3000, 4, 256)
    assert "aligned" in _err(3)
    L.bpd_dequant_q4k_gpu(None, None, -3)
    _err(2)
    L.bpd_dequant_q4k_gpu(0x1008, 0x2000, 5)
    _err(3)
    L.bpd_quant_q8_k_gpu(0x1000, 0x2000, 100)
    _err(2)
    L.bpd_quant_q8_0_gpu(0x1000, 0x2000, 33)
    _err(2)
    L.bpd_qmatmul_q8_0_dispatch_gpu(0x1000, 0x2000, 0x3000, 4, 1, 48)
    _err(2)
    L.bpd_qmatmul_q8_0_llamafile_gpu(0x1000, 0x2001, 0x3000, 4, 1, 64)
    _err(3)
    L.bpd_embed_lookup_q8_0_gpu(0x1000, None, 0x3000, 2, 64)
    _err(1)
    # measurement helpers
    L.bpdq_stream_write_gpu(0x1000, -1, 7)
    _err(2)
    L.bpdq_stream_write_gpu(0x1008, 64, 7)
    _err(3)
    L.bpdq_mfma_i8_probe_gpu(6, 10, 0x1000)
    assert "multiple of 4" in _err(2)
    L.bpdq_mfma_i8_probe_gpu(8, -1, 0x1000)
    _err(2)
    L.bpdq_mfma_i8_probe_gpu(8, 10, None)
    _err(1)
    # fused-quantization GEMVs: fp32 x must be 16-byte aligned, list sizes 0..4
    L.bpd_qmatmul_q4k_q8k_fused_gpu(0x1000, 0x2004, 0x3000, 4, 256)
    assert "x is not 16-byte aligned" in _err(3)
    L.bpd_qmatmul_q4k_q8k_fused_gpu(0x1000, 0x2000, 0x3000, 4, 200)
    _err(2)
    import ctypes
    w_arr, y_arr, m_arr = (ctypes.c_void_p * 5)(), (ctypes.c_void_p * 5)(), (ctypes.c_int * 5)()
    L.bpd_qmatmul_q4k_q8k_fused_multi_gpu(w_arr, y_arr, m_arr, 5, 0x2000, 256)
    assert "outside 0..4" in _err(2)
    m_arr[0] = 3
    w_arr[0], y_arr[0] = 0x1000, None
    L.bpd_qmatmul_q4k_q8k_fused_multi_gpu(w_arr, y_arr, m_arr, 1, 0x2000, 256)
    assert "y_list[i]" in _err(1)
    assert L.qgpu_alloc(-5) is None
    _err(2)
    L.qgpu_h2d(None, None, -1)
    _err(2)
    # the reference Python loader's per-type dequant
    L.bpd_dequant_gguf_py_gpu(0x1000, 0x2000, 256, 8)
    assert "no loader formula" in _err(2)
    L.bpd_dequant_gguf_py_gpu(0x1000, 0x2000, 300, 12)
    assert "multiple of 256" in _err(2)
    L.bpd_dequant_gguf_py_gpu(0x1000, 0x2000, 40, 2)
    assert "multiple of 32" in _err(2)
    L.bpd_dequant_gguf_py_gpu(0x1000, 0x2000, -4, 1)
    _err(2)
    L.bpd_dequant_gguf_py_gpu(None, 0x2000, 32, 2)
    _err(1)
    L.bpd_dequant_gguf_py_gpu(0x1001, 0x2008, 32, 2)
    assert "out is not 16-byte aligned" in _err(3)
    L.bpd_dequant_gguf_py_gpu(0x1001, 0x2000, 256, 14)
    assert "src is not 2-byte aligned" in _err(3)


def test_empty_calls_are_no_ops():
    L = _native.load_hip()
    L.bpd_gpu_last_error()
    L.bpd_dequant_q4k_gpu(None, None, 0)
    L.bpd_qmatmul_q4k_q8k_gpu(None, None, None, 0, 4096)
    L.bpd_quant_q8_0_gpu(None, None, 0)
    L.bpd_dequant_gguf_py_gpu(None, None, 0, 11)
    assert L.qgpu_alloc(0) is None
    assert L.bpd_gpu_last_error() == 0


def test_gpu_wrapper_raises():
    with pytest.raises(gpu.BpdqError) as e:
        gpu.call("bpd_qmatmul_q4k_gpu", None, None, None, 3, 100)
    assert e.value.code == 2


def test_synth_deterministic_and_chunk_invariant():
    L = _native.load_synth()
    k = synth.key(42, 5)
    a = np.empty(1000 * 144, np.uint8)
    b = np.empty(1000 * 144, np.uint8)
    L.bpdq_synth_q4k(a.ctypes.data, 1000, k, 0.02, 0.01, 1)
    L.bpdq_synth_q4k(b.ctypes.data, 1000, k, 0.02, 0.01, 7)
    assert np.array_equal(a, b)
    # block 500 alone equals block 500 of the run
    c = np.empty(144 * 1000, np.uint8)
    L.bpdq_synth_q4k(c.ctypes.data, 1000, k, 0.02, 0.01, 3)
    assert np.array_equal(a[500 * 144:501 * 144], c[500 * 144:501 * 144])
    x1 = synth.normal_f32(50001, synth.key(1, 1))
    assert abs(float(x1.mean())) < 0.02 and abs(float(x1.std()) - 1) < 0.02


def test_synth_distributions_match_configs():
    q = synth.q4k(4096, 256, synth.key(42, 0)).reshape(-1, 144)
    d = q[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = q[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(np.sqrt(np.mean(d ** 2)) - 0.02) < 0.002
    assert np.all(dm >= 0) and abs(np.sqrt(np.mean(dm ** 2)) - 0.01) < 0.001
    w = synth.q8_0(4096, 32, synth.key(42, 1)).reshape(-1, 34)
    v = w[:, 2:].view(np.int8)
    assert v.min() == -127 and v.max() == 127
    assert formats.q4k_bytes(14336, 4096) == 33030144


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_decode_step_validation_before_launch():
    """generate_token / bpd_llama_step_gpu reject bad structs before any HIP call."""
    import ctypes

    from bpd_substrate_amd import llama

    L = _native.load_hip()
    L.bpd_gpu_last_error()
    assert L.generate_token(None, None, None, None, 0, None, None, None, None, 64, 100) == -1
    assert "cfg is NULL" in _err(1)
    cfg = llama.ModelConfig(1, 256, 4, 2, 64, 512, 100, 64, 1e-5, 10000.0)
    bufs = llama.WorkBuffers(*[0x10000 * (i + 1) for i in range(11)])
    a = (ctypes.addressof(cfg), ctypes.addressof(bufs))
    for field, val, text in (("head_dim", 48, "head_dim"), ("n_head_kv", 3, "n_head_kv"), ("max_seq", 0, "max_seq"),
                             ("n_embd", 320, "n_embd")):
        old = getattr(cfg, field)
        setattr(cfg, field, val)
        assert L.generate_token(None, a[0], a[1], None, 0, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
        assert text in _err(2)
        setattr(cfg, field, old)
    assert L.generate_token(None, a[0], a[1], None, 64, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
    assert "position" in _err(2)
    assert L.generate_token(None, a[0], a[1], None, 0, 0x1000, 0x2000, None, None, 256, 100) == -1
    assert "lm_f32" in _err(1)
    bufs.k = 0x10004
    assert L.generate_token(None, a[0], a[1], None, 0, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
    assert "buf.k is not 16-byte aligned" in _err(3)
    bufs.k = 0x20000
    assert L.generate_token(None, a[0], a[1], None, 0, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
    assert "layers is NULL" in _err(1)
    lw = (llama.LayerWeights * 1)()
    kp = (ctypes.c_void_p * 1)(0x40000)
    kv = llama.KVCache(ctypes.cast(kp, ctypes.POINTER(ctypes.c_void_p)), ctypes.cast(kp, ctypes.POINTER(ctypes.c_void_p)))
    assert L.generate_token(ctypes.addressof(lw), a[0], a[1], ctypes.addressof(kv), 0, 0x1000, 0x2000, 0x3000, None,
                            256, 100) == -1
    assert "layer 0 q is 0 x 0" in _err(2)
    assert L.bpd_llama_step_gpu(7, None, a[0], a[1], None, 0, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
    assert "weight_format" in _err(2)
    cfg.n_embd, cfg.n_head = 256, 4
    assert L.bpd_llama_step_gpu(llama.W_Q4K, None, a[0], a[1], None, 0, 0x1000, 0x2000, 0x3000, None, 256, 100) == -1
    assert "ff_dim" not in _err(1)
    L.bpd_residual_rmsnorm_gpu(0x1000, None, None, 0x2000, None, None, 48, 1e-5)
    assert "multiple of 32" in _err(2)
    assert L.gpu_alloc(-1) is None
    _err(2)


def test_tensor_helpers_check_buffer_sizes():
    """The C ABI takes bare pointers, so the torch helpers check sizes on the host and
    raise before any launch (CPU tensors: nothing here reaches the GPU)."""
    import torch

    w = torch.zeros(4 * 144, dtype=torch.uint8)            # 4 Q4_K blocks
    xq = torch.zeros(292, dtype=torch.uint8)               # one Q8_K block
    with pytest.raises(gpu.BpdqError, match="w holds 576 bytes, the call needs 1152"):
        gpu.qmatmul_q4k_q8k(w, xq, 8, 256)
    with pytest.raises(gpu.BpdqError, match="xq holds"):
        gpu.qmatmul_q4k_q8k(torch.zeros(8 * 2 * 144, dtype=torch.uint8), xq, 8, 512)
    with pytest.raises(gpu.BpdqError, match="out holds"):
        gpu.qmatmul_q4k_q8k(torch.zeros(8 * 144, dtype=torch.uint8), xq, 8, 256, out=torch.zeros(7))
    with pytest.raises(gpu.BpdqError, match="not contiguous"):
        gpu.qmatmul_q4k(w, torch.zeros(512)[::2], 4, 256)
    with pytest.raises(gpu.BpdqError, match="Xq holds"):
        gpu.qmatmul_q8_0_dispatch(torch.zeros(4 * 34, dtype=torch.uint8), torch.zeros(33, dtype=torch.uint8), 4, 1, 32)
    with pytest.raises(gpu.BpdqError, match="X holds"):
        gpu.qmatmul_q8_0_llamafile(torch.zeros(4 * 34, dtype=torch.uint8), torch.zeros(31), 4, 1, 32)
    with pytest.raises(gpu.BpdqError, match=r"w\[1\] holds"):
        gpu.qmatmul_q4k_q8k_multi([w, w], xq, [4, 5], 256)
    with pytest.raises(gpu.BpdqError, match="w holds"):
        gpu.qmatmul_q6k_q8k(torch.zeros(210, dtype=torch.uint8), xq, 2, 256)


def test_call_refuses_names_without_a_signature():
    # ctypes without argtypes passes Python ints as 32-bit C ints: a device pointer would
    # arrive cut to its low 32 bits, so gpu.call only calls declared entry points
    with pytest.raises(KeyError, match="no ctypes signature"):
        gpu.call("bpd_not_declared_anywhere_gpu", 0x7F1234561000)


def test_p_order_k_limit_is_refused_before_launch():
    L = _native.load_hip()
    L.bpd_gpu_last_error()
    L.bpd_qdot_q8_0_q8_0_grid_gpu(0x1000, 0x2000, 0x3000, 1, 8, 52416 + 32)
    assert "52416" in _err(7)
    L.bpd_qmatmul_q8_0_gpu(0x1000, 0x2000, 0x3000, 1, 8, 52416 + 32)
    _err(7)
    L.bpd_qmm_q4k_gpu(0x1000, 0x2000, 0x3000, 2, 3, 300)
    assert "multiple of 256" in _err(2)
