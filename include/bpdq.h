/* bpdq.h — C ABI of libbpdq_hip.so, the gfx950 (MI355X) implementation of the
 * bpd-substrate quantized-inference path.
 *
 * Conventions, kept from the reference's ctypes surface:
 *   - every tensor argument is a device pointer (qgpu_alloc, hipMalloc, or a
 *     torch-ROCm tensor's data_ptr()); sizes are C int; functions return void;
 *   - GGUF block bytes are consumed unchanged: Q4_K 144 B / 256 elements,
 *     Q8_0 34 B / 32 elements, rows stored with K contiguous;
 *   - kernels are launched asynchronously on the current stream (the null
 *     stream unless bpd_gpu_set_stream() chose another), like the reference's
 *     <<<grid, block>>> launches; qgpu_h2d/qgpu_d2h are synchronous copies.
 * Unlike the reference, every entry point validates its arguments first.  A
 * NULL pointer with a non-empty size, a negative size, K that is not a multiple
 * of the block length, or a misaligned pointer launches nothing, leaves the
 * outputs untouched and records an error code readable with bpd_gpu_last_error().
 * Pointer alignment required: Q4_K tensors 16 B; fp32 vectors of
 * bpd_quant_q8_k_gpu 16 B; every other fp32 / Q8_K pointer 4 B; Q8_0 bytes 1 B.
 *
 * Citations are /root/reference/<file>:<line> of the interface each entry
 * point replaces.
 */
#ifndef BPDQ_H
#define BPDQ_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error reporting (no counterpart in the reference, whose CUDA calls are
 *      never checked: bench/bpd_quant_gpu.cu:162-176) ---------------------- */
#define BPDQ_OK 0
#define BPDQ_ERR_NULL 1   /* NULL pointer for a non-empty tensor */
#define BPDQ_ERR_SHAPE 2  /* negative size or K not a multiple of the block length */
#define BPDQ_ERR_ALIGN 3  /* pointer alignment below what the kernel loads with */
#define BPDQ_ERR_HIP 4    /* the HIP runtime reported an error (launch, copy, sync) */
#define BPDQ_ERR_ALLOC 5  /* device allocation failed */
#define BPDQ_ERR_CAPTURE 6 /* the stream's workspace would have to grow during stream capture:
                              make the same call once outside capture, on the same stream */
#define BPDQ_ERR_LIMIT 7   /* the call needs more than a fixed-size buffer holds */
/* First error recorded on the calling thread since the previous call; clears it. */
int bpd_gpu_last_error(void);
/* Text of the most recent error on the calling thread ("" if none). */
const char* bpd_gpu_last_error_message(void);
/* Launch stream for every later call (a hipStream_t; NULL = the null stream). */
void bpd_gpu_set_stream(void* hip_stream);
/* No counterpart in the reference (its CPU functions malloc per call).  The
 * entry points that quantize fp32 activations keep them in a device workspace
 * owned by the library, one per (device, stream), at most 64 at once.  A
 * workspace only grows, and a buffer it outgrows is kept, not freed: a HIP graph
 * captured with it may still replay into it.  This call frees every buffer of
 * (current device, hip_stream) after waiting for the whole device to go idle,
 * and frees the stream's slot of the 64.  Call it before destroying a stream
 * that library calls ran on, and only once no captured graph that holds
 * library calls made on that stream will be replayed again. */
void bpd_gpu_workspace_release(void* hip_stream);

/* ---- Q4_K: bench/bpd_quant_gpu.cu:160-178 ------------------------------- */
/* out[256 b + e] = dequant of Q4_K block b in the bpd element map
 * (bench/bpd_quant_gpu.cu:162-164, math of bench/bpd_quant.c:41-81); 0 ULP. */
void bpd_dequant_q4k_gpu(const uint8_t* q_dev, float* out_dev, int n_blocks);
/* y[M] = W_q4k[M,K] x_f32[K] with the reference CPU order of bench/bpd_quant.c:88-109
 * (a sequential fp32 chain per row): bit-identical to bpd_qmatmul_q4k.
 * Replaces bench/bpd_quant_gpu.cu:166-169. */
void bpd_qmatmul_q4k_gpu(const uint8_t* w_dev, const float* x_dev, float* y_dev, int M, int K);
void* qgpu_alloc(int bytes);                                  /* bench/bpd_quant_gpu.cu:172 */
void qgpu_free(void* p);                                      /* :173 */
void qgpu_h2d(void* dst_dev, const void* src_host, int bytes); /* :174 */
void qgpu_d2h(void* dst_host, const void* src_dev, int bytes); /* :175 */
void qgpu_sync(void);                                         /* :176 */

/* ---- aliases of the launch-sweep library, bench/bpd_quant_gpu_sweep.cu:131-151.
 * All eight produce the full bpd-order dequant (the reference's v1<128/64/32>
 * left elements unwritten, bench/bpd_quant_gpu_sweep.cu:39-41). */
void dequant_v1_256(const uint8_t* q, float* o, int nb);
void dequant_v1_128(const uint8_t* q, float* o, int nb);
void dequant_v1_64(const uint8_t* q, float* o, int nb);
void dequant_v1_32(const uint8_t* q, float* o, int nb);
void dequant_ilp2(const uint8_t* q, float* o, int nb);
void dequant_multi2(const uint8_t* q, float* o, int nb);
void dequant_multi4(const uint8_t* q, float* o, int nb);
void dequant_multi8(const uint8_t* q, float* o, int nb);
void* sgpu_alloc(int bytes);
void sgpu_free(void* p);
void sgpu_h2d(void* d, const void* s, int bytes);
void sgpu_d2h(void* d, const void* s, int bytes);
void sgpu_sync(void);

/* ---- aliases of the head-to-head library, bench/bench_dequant_gpu_h2h.cu:74-82:
 * GGUF (llama.cpp) element map with that file's f16 decode. */
void run_llamacpp(const void* q, float* o, int nb);
void run_bpd(const void* q, float* o, int nb);
void* galloc(int bytes);
void gfree(void* p);
void gh2d(void* d, const void* s, int bytes);
void gd2h(void* d, const void* s, int bytes);
void gsync(void);

/* ---- new Q4_K / Q8_K entry points (the reference has no Q8_K code:
 *      docs/llama-kernel-audit.md:65; block size lib/gguf_emit_manifest.pl:142) */
/* GGUF element map (bench/bench_dequant_gpu_h2h.cu:27-48). */
void bpd_dequant_q4k_gguf_gpu(const uint8_t* q_dev, float* out_dev, int n_blocks);
/* x[n] fp32 -> n/256 Q8_K blocks {f32 d; i8 qs[256]; i16 bsums[16]} (292 B). */
void bpd_quant_q8_k_gpu(const float* x_dev, uint8_t* y_q8k_dev, int n);
/* y[M] = W_q4k[M,K] . x_q8k[K]: exact integer sub-block sums, fixed fp32 tree
 * (bpd element map / GGUF element map). */
void bpd_qmatmul_q4k_q8k_gpu(const uint8_t* w_dev, const uint8_t* xq8k_dev, float* y_dev, int M, int K);
void bpd_qmatmul_q4k_q8k_gguf_gpu(const uint8_t* w_dev, const uint8_t* xq8k_dev, float* y_dev, int M, int K);

/* n (0..4) Q4_K matrices sharing one Q8_K activation, in one launch: y_list[i][M_list[i]] =
 * W_i . xq8k, each bit-identical to bpd_qmatmul_q4k_q8k_gpu on that matrix.  w_list, y_list and
 * M_list are host arrays (of device pointers).  For the Q/K/V and gate/up GEMVs of a decode step
 * (bench/bpd_cpu.c:5642-5727 issues them as separate calls). */
void bpd_qmatmul_q4k_q8k_multi_gpu(const uint8_t* const* w_list, float* const* y_list, const int* M_list, int n,
                                   const uint8_t* xq8k_dev, int K);

/* The two above with the activation given as fp32 x[K] (16-byte aligned): the kernel quantizes x
 * to Q8_K itself, so y is bit-identical to bpd_quant_q8_k_gpu followed by
 * bpd_qmatmul_q4k_q8k_gpu / _multi_gpu, in one launch instead of two.  For a decode step, which
 * re-quantizes every activation before its GEMVs (bench/bpd_cpu.c:5642-5733 quantizes inside
 * each bpd_qmatmul_q8_0_llamafile_cpu call, bench/bpd_cpu.c:4429-4452). */
void bpd_qmatmul_q4k_q8k_fused_gpu(const uint8_t* w_dev, const float* x_dev, float* y_dev, int M, int K);
void bpd_qmatmul_q4k_q8k_fused_multi_gpu(const uint8_t* const* w_list, float* const* y_list, const int* M_list,
                                         int n, const float* x_dev, int K);

/* ---- the padded Q8 weight layout of the reference's dp4a GPU path ----
 * fp32 x[N][K] -> [K/32][N][64] bytes, record (b, n) = {f16 d, 0, 0, int8 q[32], 28 zero bytes}
 * with d = RN(max(amax, 1e-10)/127) and q = clip(round-half-even(RN(x/d)), -128, 127):
 * q8_pad64_coalesced (inference/llamatov_c_inference.py:88-100), done on the GPU at load time. */
void bpd_q8_pad64_from_f32_gpu(const float* x_dev, uint8_t* out_dev, int N, int K);
/* The Q8_0 tile-order T product (bpd_qmatmul_q8_0_dispatch_gpu) with W in that layout:
 * out[token * m_weight + row], bit-identical to the dispatcher on the same (d, q) in 34-byte
 * Q8_0 rows.  Xq: m_tokens rows of Q8_0 blocks. */
void bpd_qmatmul_q8_pad64_gpu(const uint8_t* W_pad64_dev, const uint8_t* Xq_dev, float* out_dev, int m_weight,
                              int m_tokens, int K);

/* ---- Q6_K (210-byte blocks: ql[128], qh[64], int8 sc[16], f16 d) ----
 * The reference has Q6_K only as Python: inference/llamatov_helpers.py:161-179 dequantizes
 * it to fp32, with its own element map (element 2i / 2i+1 = low / high nibble of ql[i],
 * element 4j+k = bits 2k..2k+1 of qh[j]).  The _gguf_ forms use the GGUF (llama.cpp
 * dequantize_row_q6_K) map.  Q6_K pointers need 2-byte alignment. */
void bpd_dequant_q6k_gpu(const uint8_t* q_dev, float* out_dev, int n_blocks);
void bpd_dequant_q6k_gguf_gpu(const uint8_t* q_dev, float* out_dev, int n_blocks);
/* y[M] = W_q6k[M,K] . x_q8k[K]: exact integer group sums, then the fp32 order of
 * bpd_qmatmul_q4k_q8k_gpu (no reference code: the reference never multiplies Q6_K
 * without dequantizing it first). */
void bpd_qmatmul_q6k_q8k_gpu(const uint8_t* w_dev, const uint8_t* xq8k_dev, float* y_dev, int M, int K);
void bpd_qmatmul_q6k_q8k_gguf_gpu(const uint8_t* w_dev, const uint8_t* xq8k_dev, float* y_dev, int M, int K);

/* ---- the reference Python loader's fp32 of a GGUF tensor ----
 * load_tensor_by_type (inference/llamatov_helpers.py:196-222) on the device: out[n_elements] in
 * fp32 from the tensor's bytes, with the Python's formulas, element maps and float32 operation
 * order, NaN bits as numpy gives them on x86.  ggml_type: 0 F32, 1 F16 (astype, :205-207),
 * 2 Q4_0 (:71-98), 10 Q2_K (:25-39), 11 Q3_K (the reference's approximate form, :42-68),
 * 12 Q4_K (its own element map, :101-158), 14 Q6_K (:161-179, as bpd_dequant_q6k_gpu).
 * The reference returns zeros for any other type; here that is BPDQ_ERR_SHAPE, nothing written.
 * n_elements a multiple of the type's block (1, 32 or 256); out 16-byte aligned; src any
 * alignment (2 bytes for Q6_K). */
void bpd_dequant_gguf_py_gpu(const uint8_t* src_dev, float* out_dev, int64_t n_elements, int ggml_type);

/* ---- Q8_0 on the GPU, same signatures as the CPU functions they mirror ---- */
void bpd_dequant_q8_0_gpu(const uint8_t* raw_dev, float* out_dev, int n_blocks);           /* bench/bpd_cpu.c:3960 */
/* ids must index rows of the table (0 <= id < rows); bench/bpd_cpu.c:4002 */
void bpd_embed_lookup_q8_0_gpu(const uint8_t* table_dev, const int32_t* ids_dev, float* out_dev, int n_tokens,
                               int embed_dim);
void bpd_quant_q8_0_gpu(const float* x_dev, uint8_t* y_dev, int n_elements);                /* bench/bpd_cpu.c:4106 */
/* out[token * m_weight + row], AVX1 llamafile tile order: bit-identical to
 * bpd_qmatmul_q8_0_dispatch_cpu of the -mavx build (bench/bpd_gemm_q8_0_cpu.c:159). */
void bpd_qmatmul_q8_0_dispatch_gpu(const uint8_t* Wq_dev, const uint8_t* Xq_dev, float* out_dev, int m_weight,
                                   int m_tokens, int K);
/* quantize X (fp32, m_tokens x K) then the dispatcher (bench/bpd_cpu.c:4429-4452).
 * The Q8_0 rows of X go to a device workspace owned by the library, one per
 * (device, stream), grown on demand (buffers it outgrows are kept for graphs
 * captured with them, see bpd_gpu_workspace_release); growth fails with
 * BPDQ_ERR_CAPTURE during stream capture.  Calls on one stream may come from
 * several host threads. */
void bpd_qmatmul_q8_0_llamafile_gpu(const uint8_t* W_dev, const float* X_dev, float* out_dev, int m_weight,
                                    int m_tokens, int K);

/* No counterpart in the reference: bpd_qmatmul_q8_0_llamafile_gpu for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and bits; the Q8_0 rows of X go to a fixed 8 MiB device array
 * that each GPU holds for the life of the process, so the call allocates nothing.
 * m_tokens * (K/32) * 34 bytes above 8 MiB are refused with BPDQ_ERR_LIMIT, nothing launched.
 * Every call on one GPU shares that array: calls that overlap on one GPU (other streams,
 * other host threads) race on it. */
void bpd_qmatmul_q8_0_llamafile_noalloc_gpu(const uint8_t* W_dev, const float* X_dev, float* out_dev, int m_weight,
                                            int m_tokens, int K);

/* Same cells in the scalar order S (bench/bpd_gemm_q8_0_cpu.c:102-131): bit-identical
 * to bpd_qmatmul_q8_0_dispatch_cpu / _llamafile_cpu of the -O2 (non-AVX) build.  Runs
 * on int8 MFMA (one 32x32x32 step per Q8_0 block) with an fp32 epilogue per block:
 * the batched-prefill GEMM (cfg4: 512 tokens x 4096 x 14336 rows). */
void bpd_qmatmul_q8_0_dispatch_s_gpu(const uint8_t* Wq_dev, const uint8_t* Xq_dev, float* out_dev, int m_weight,
                                     int m_tokens, int K);
void bpd_qmatmul_q8_0_llamafile_s_gpu(const uint8_t* W_dev, const float* X_dev, float* out_dev, int m_weight,
                                      int m_tokens, int K);

/* ---- the reference's other CPU forms on the GPU ----
 * bpd_qmm_q4k (bench/bpd_quant.c:114-137): C[M][N] = dequant(A_q4k[M][K]) . B[K][N], B and C
 * row-major fp32; each cell the reference's sequential chain from +0.0 over k in element
 * order: bit-identical to bpd_qmm_q4k, NaN bits included.  A 16-byte aligned. */
void bpd_qmm_q4k_gpu(const uint8_t* A_dev, const float* B_dev, float* C_dev, int M, int N, int K);
/* bpd_qdot_q8_0_q8_0_cpu (bench/bpd_cpu.c:4208-4259, the AVX1 build's pair order P) for every
 * (activation row m, weight row n): out[m * N + n] = qdot(Wq row n, Xq row m, K/32).  Wq: N
 * Q8_0 rows, Xq: M Q8_0 rows, of K/32 blocks each.  Bit-identical over the whole int8 range
 * (the SSSE3 maddubs arithmetic is reproduced for -128 quants).  K <= 52,416. */
void bpd_qdot_q8_0_q8_0_grid_gpu(const uint8_t* Wq_dev, const uint8_t* Xq_dev, float* out_dev, int M, int N, int K);
/* The same cells in the scalar build's order S (bench/bpd_cpu.c:4263-4280), NaN bits included. */
void bpd_qdot_q8_0_q8_0_grid_s_gpu(const uint8_t* Wq_dev, const uint8_t* Xq_dev, float* out_dev, int M, int N,
                                   int K);
/* bpd_qmatmul_q8_0_cpu(W, X, out, M = tokens, N = weight rows, K) (bench/bpd_cpu.c:4295-4315):
 * quantize the M fp32 rows of X to Q8_0 (bpd_quant_q8_0_cpu), then out[m * N + n] = qdot:
 * order P (the -mavx build) and order S (the -O2 build).  X 4-byte aligned; the quantized rows
 * go to the stream's workspace.  The P form needs K <= 52,416. */
void bpd_qmatmul_q8_0_gpu(const uint8_t* W_dev, const float* X_dev, float* out_dev, int M, int N, int K);
void bpd_qmatmul_q8_0_s_gpu(const uint8_t* W_dev, const float* X_dev, float* out_dev, int M, int N, int K);

/* ---- the prefill's fused gate/up (no counterpart in the reference) ----------
 * Order S (as bpd_qdot_q8_0_q8_0_grid_s_gpu) for the M Q8_0 rows of Xq against the F rows of
 * Wg and of Wu, then y = silu(g) * u (bpd_swiglu_fuse_cpu, bench/bpd_cpu.c:5504-5507) and its
 * Q8_0 rows (bpd_quant_q8_0_cpu) into yq: M rows of F/32 blocks, as the multi-token block
 * feeds its down projection.  F a multiple of 64, K of 128; Wg, Wu and Xq 4-byte aligned. */
void bpdq_q8_0_gemm_swiglu_s_gpu(const uint8_t* Wg_dev, const uint8_t* Wu_dev, const uint8_t* Xq_dev,
                                 uint8_t* yq_dev, int M, int F, int K);

/* ---- measurement helper (no counterpart in the reference) -------------------
 * Reads n16 16-byte chunks at p once, as fast as a plain streaming kernel can,
 * and writes *sink only if the data XORs to a magic value.  bench.py uses it for
 * the single-launch HBM read floor of a given size, and it is the known-traffic
 * kernel that calibrates rocprofv3's FETCH_SIZE counter. */
void bpdq_stream_read_gpu(const uint8_t* p, int n16, uint32_t* sink);
/* Writes n16 16-byte chunks at p once (non-temporal stores of a pattern derived
 * from value): the single-launch HBM write floor of a given size. */
void bpdq_stream_write_gpu(uint8_t* p, int n16, uint32_t value);
/* waves (a multiple of 4) waves each run iters rounds of 4 register-only
 * v_mfma_i32_32x32x32_i8 (262,144 int8 ops per round); *sink is written only
 * if the result folds to a magic value.  The device's int8 MFMA rate. */
void bpdq_mfma_i8_probe_gpu(int waves, int iters, uint32_t* sink);

#ifdef __cplusplus
}
#endif
#endif /* BPDQ_H */
