"""Loading of the in-tree native libraries, with ctypes signatures.

The argtypes follow the reference's own ctypes declarations (every pointer
c_void_p, every size c_int, void returns): bench/verify_quant_gpu.py:27-42,
bench/bench_gpu_sweep.py:6-20, bench/bench_dequant_gpu_h2h.py:5-13,
bench/test_gemm_q8_0_tiles.py:42-69.
There is no fallback: if libbpdq_hip.so is missing the import of the GPU entry
points fails with an error naming the build command.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
# BPDQ_HIP_LIB / BPDQ_SYNTH_LIB name other builds of the same libraries (the CPU
# test suite's sanitized host-only build); unset, the in-tree builds are used.
HIP_LIB = os.environ.get("BPDQ_HIP_LIB") or os.path.join(PKG, "libbpdq_hip.so")
SYNTH_LIB = os.environ.get("BPDQ_SYNTH_LIB") or os.path.join(PKG, "libbpdq_synth.so")

P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float

# name -> (restype, argtypes); the full exported surface of include/bpdq.h
HIP_SIGNATURES = {
    "bpd_gpu_last_error": (I, []),
    "bpd_gpu_last_error_message": (ctypes.c_char_p, []),
    "bpd_gpu_set_stream": (None, [P]),
    "bpd_gpu_workspace_release": (None, [P]),
    "bpd_dequant_q4k_gpu": (None, [P, P, I]),
    "bpd_qmatmul_q4k_gpu": (None, [P, P, P, I, I]),
    "qgpu_alloc": (P, [I]),
    "qgpu_free": (None, [P]),
    "qgpu_h2d": (None, [P, P, I]),
    "qgpu_d2h": (None, [P, P, I]),
    "qgpu_sync": (None, []),
    "dequant_v1_256": (None, [P, P, I]),
    "dequant_v1_128": (None, [P, P, I]),
    "dequant_v1_64": (None, [P, P, I]),
    "dequant_v1_32": (None, [P, P, I]),
    "dequant_ilp2": (None, [P, P, I]),
    "dequant_multi2": (None, [P, P, I]),
    "dequant_multi4": (None, [P, P, I]),
    "dequant_multi8": (None, [P, P, I]),
    "sgpu_alloc": (P, [I]),
    "sgpu_free": (None, [P]),
    "sgpu_h2d": (None, [P, P, I]),
    "sgpu_d2h": (None, [P, P, I]),
    "sgpu_sync": (None, []),
    "run_llamacpp": (None, [P, P, I]),
    "run_bpd": (None, [P, P, I]),
    "galloc": (P, [I]),
    "gfree": (None, [P]),
    "gh2d": (None, [P, P, I]),
    "gd2h": (None, [P, P, I]),
    "gsync": (None, []),
    "bpd_dequant_q4k_gguf_gpu": (None, [P, P, I]),
    "bpd_quant_q8_k_gpu": (None, [P, P, I]),
    "bpd_qmatmul_q4k_q8k_gpu": (None, [P, P, P, I, I]),
    "bpd_qmatmul_q4k_q8k_gguf_gpu": (None, [P, P, P, I, I]),
    "bpd_qmatmul_q4k_q8k_multi_gpu": (None, [P, P, P, I, P, I]),
    "bpd_qmatmul_q4k_q8k_fused_gpu": (None, [P, P, P, I, I]),
    "bpd_q8_pad64_from_f32_gpu": (None, [P, P, I, I]),
    "bpd_qmatmul_q8_pad64_gpu": (None, [P, P, P, I, I, I]),
    "bpd_dequant_q6k_gpu": (None, [P, P, I]),
    "bpd_dequant_gguf_py_gpu": (None, [P, P, ctypes.c_int64, I]),
    "bpd_dequant_q6k_gguf_gpu": (None, [P, P, I]),
    "bpd_qmatmul_q6k_q8k_gpu": (None, [P, P, P, I, I]),
    "bpd_qmatmul_q6k_q8k_gguf_gpu": (None, [P, P, P, I, I]),
    "bpd_qmatmul_q4k_q8k_fused_multi_gpu": (None, [P, P, P, I, P, I]),
    "bpd_dequant_q8_0_gpu": (None, [P, P, I]),
    "bpd_embed_lookup_q8_0_gpu": (None, [P, P, P, I, I]),
    "bpd_quant_q8_0_gpu": (None, [P, P, I]),
    "bpd_qmatmul_q8_0_dispatch_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_llamafile_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_llamafile_noalloc_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmm_q4k_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qdot_q8_0_q8_0_grid_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qdot_q8_0_q8_0_grid_s_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_s_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_dispatch_s_gpu": (None, [P, P, P, I, I, I]),
    "bpd_qmatmul_q8_0_llamafile_s_gpu": (None, [P, P, P, I, I, I]),
    "bpdq_q8_0_gemm_swiglu_s_gpu": (None, [P, P, P, P, I, I, I]),
    "bpdq_stream_read_gpu": (None, [P, I, P]),
    "bpdq_stream_write_gpu": (None, [P, I, ctypes.c_uint32]),
    "bpdq_mfma_i8_probe_gpu": (None, [I, I, P]),
    # include/bpdq_llama.h; the struct arguments are passed by address
    # (inference/llamatov_c_inference.py:66-83 declares them POINTER(struct))
    "generate_token": (I, [P, P, P, P, I, P, P, P, P, I, I]),
    "gpu_alloc": (P, [I]),
    "gpu_copy_h2d": (None, [P, P, I]),
    "gpu_copy_d2h": (None, [P, P, I]),
    "gpu_sync": (None, []),
    "gpu_free": (None, [P]),
    "bpd_llama_step_gpu": (I, [I, P, P, P, P, I, P, P, P, P, I, I]),
    "bpd_llama_step_ext_gpu": (I, [I, P, P, P, P, P, I, P, P, P, P, I, I]),
    # bench/bpd_llamatov_infer.py:459-466 binds bpd_llama_forward_cpu with these argtypes
    "bpd_llama_block_gpu": (None, [P, P, P, P, I, I, P, P, P, P, P, P]),
    "bpd_llama_block_s_gpu": (None, [P, P, P, P, I, I, P, P, P, P, P, P]),
    "bpd_llama_forward_gpu": (None, [P, I, P, P, P, I, P, P, P, P]),
    "bpd_llama_forward_s_gpu": (None, [P, I, P, P, P, I, P, P, P, P]),
    "bpd_residual_rmsnorm_gpu": (None, [P, P, P, P, P, P, I, F]),
    "bpd_expf_gpu": (None, [P, P, I]),
    "bpd_argmax_gpu": (None, [P, I, P]),
}

SYNTH_SIGNATURES = {
    "bpdq_synth_key": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
    "bpdq_synth_q4k": (None, [P, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, I]),
    "bpdq_synth_q8_0": (None, [P, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double, I]),
    "bpdq_synth_normal_f32": (None, [P, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double, I]),
    "bpdq_synth_bytes": (None, [P, ctypes.c_int64, ctypes.c_uint64, I]),
}

_cache = {}


def _load(path, sigs, what):
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{what} is not built ({path} missing): run `python -m bpd_substrate_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[path] = lib
    return lib


def load_hip():
    """The gfx950 library (libbpdq_hip.so). Raises if it has not been built."""
    return _load(HIP_LIB, HIP_SIGNATURES, "libbpdq_hip.so")


def load_synth():
    return _load(SYNTH_LIB, SYNTH_SIGNATURES, "libbpdq_synth.so")
