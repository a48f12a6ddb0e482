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
