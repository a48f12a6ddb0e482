"""GGUF block layouts used on the path (byte-for-byte the reference's).

Q4_K: {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]} = 144 B / 256 elements
      (/root/reference/bench/bpd_quant.c:15-22, bench/bench_dequant_gpu_h2h.cu:12)
Q8_0: {f16 d; i8 qs[32]} = 34 B / 32 elements (bench/bpd_cpu.c:3886-3888)
Q8_K: {f32 d; i8 qs[256]; i16 bsums[16]} = 292 B / 256 elements (size from
      lib/gguf_emit_manifest.pl:142; field order is llama.cpp's)
Rows are stored with K contiguous: row r of an M x K matrix starts at
r * (K / block_elems) * block_bytes.
"""

Q4K_ELEMS, Q4K_BYTES = 256, 144
Q8_0_ELEMS, Q8_0_BYTES = 32, 34
Q8K_ELEMS, Q8K_BYTES = 256, 292

# element maps of a Q4_K block (which nibble feeds which element)
ORDER_BPD = 0   # bench/bpd_quant.c:68-72
ORDER_GGUF = 1  # bench/bench_dequant_gpu_h2h.cu:31-46


def q4k_bytes(rows: int, k: int) -> int:
    return rows * (k // Q4K_ELEMS) * Q4K_BYTES


def q8_0_bytes(rows: int, k: int) -> int:
    return rows * (k // Q8_0_ELEMS) * Q8_0_BYTES


def q8k_bytes(rows: int, k: int) -> int:
    return rows * (k // Q8K_ELEMS) * Q8K_BYTES


PAD64_BYTES = 64  # record {f16 d, 0, 0, i8 q[32], 28 zero bytes}


def q8_0_rows_to_pad64(rows, n: int, k: int):
    """Q8_0 rows [n][k/32][34] -> the padded layout [k/32][n][64] of
    q8_pad64_coalesced (inference/llamatov_c_inference.py:88-100): a byte
    relayout of the same (d, q) pairs, so a GGUF Q8_0 tensor feeds
    generate_token without requantization."""
    import numpy as np

    nb = k // Q8_0_ELEMS
    src = np.asarray(rows, dtype=np.uint8).reshape(n, nb, Q8_0_BYTES)
    out = np.zeros((nb, n, PAD64_BYTES), np.uint8)
    out[:, :, 0:2] = src[:, :, 0:2].transpose(1, 0, 2)
    out[:, :, 4:36] = src[:, :, 2:34].transpose(1, 0, 2)
    return out.reshape(-1)
