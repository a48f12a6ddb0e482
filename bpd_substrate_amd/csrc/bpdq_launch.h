// bpdq_launch.h — host-side launchers of the gfx950 kernels (internal to
// libbpdq_hip.so; the exported C ABI is include/bpdq.h).  Callers have already
// validated every argument: shapes, multiples, pointer alignment.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace bpdq {

// A device workspace of at least the requested size for launches on stream s,
// locked for the caller until the lease is destroyed (after its launches are
// enqueued).  ptr is nullptr, with the error recorded, when it cannot be had:
// allocation failure, or growth requested during stream capture
// (BPDQ_ERR_CAPTURE).
struct WsLease {
    std::unique_lock<std::mutex> lock;
    void* ptr = nullptr;
};
WsLease workspace(size_t bytes, hipStream_t s, const char* fn);

// Error recording (read back with bpd_gpu_last_error) and the launch stream of
// the exported ABI, for entry points defined outside abi.hip.
void abi_error(int code, const char* fn, const char* what);
bool abi_hip_ok(hipError_t e, const char* fn);
hipStream_t abi_stream();

void launch_dequant_q4k(const uint8_t* q, float* out, int n_blocks, int order, hipStream_t s);
void launch_qmatmul_q4k_chain(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t s);
void launch_quant_q8k(const float* x, uint8_t* y, int n, hipStream_t s);
void launch_qmatmul_q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s);

void launch_qmatmul_q4k_q8k_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const uint8_t* xq,
                                  int K, int order, hipStream_t s);
// The fused-quantization GEMV handles K <= fused_max_k(); beyond it callers
// quantize into a buffer and use launch_qmatmul_q4k_q8k_multi.
int fused_max_k();
void launch_qmatmul_q4k_fused_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const float* x,
                                    int K, int order, hipStream_t s);
// Gate and up (M rows each, K <= fused_max_k()) with the fp32 activation x:
// y[r] = silu(gate_r) * up_r, gate_r and up_r as the fused GEMV computes them.
void launch_qmatmul_q4k_fused_swiglu(const uint8_t* w_gate, const uint8_t* w_up, float* y, int M, const float* x,
                                     int K, int order, hipStream_t s);
// The same from a Q8_K activation xq (K <= 4096).
void launch_qmatmul_q4k_swiglu_q8k(const uint8_t* w_gate, const uint8_t* w_up, float* y, int M, const uint8_t* xq,
                                   int K, int order, hipStream_t s);

// The decode step's RMSNorm folded into its GEMVs (n_embd = 4096, ff 4096 or
// 14336, Q4_K weights 16-byte aligned; norm_fusion_fits): the producer (O,
// down) adds its rows into the residual row x and writes one binary64 partial
// sum of squares per workgroup; the consumer turns them into the norm's scale:
// the Q/K/V GEMV quantizes h = (x * scale) * w itself, the gate/up GEMV reads
// the Q8_K of h that one small kernel writes (a 14336-row GEMV repeating the
// norm in each of its 3584 workgroups measured 19.7 us against 11.0 + 4.6).
struct NormIn {
    const float* x;
    const float* w;
    const double* part;
    int npart;
    float eps;
};
struct ResOut {
    float* x;
    double* part;
};
bool norm_fusion_fits(int n_embd, int ff);
void launch_q4k_norm_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const NormIn& nin,
                           int order, hipStream_t s);
int launch_q4k_res(const uint8_t* w, int M, const float* x, int K, const ResOut& ro, int order, hipStream_t s);

void launch_dequant_q6k(const uint8_t* q, float* out, int n_blocks, int order, hipStream_t s);
// the reference Python loader's fp32 of a GGUF tensor (gguf_py.hip); false for a
// type it has no formula for
bool launch_dequant_gguf_py(const uint8_t* src, float* out, int64_t n_elements, int ggml_type, hipStream_t s);
void launch_qmatmul_q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s);

void launch_dequant_q8_0(const uint8_t* raw, float* out, int n_blocks, hipStream_t s);
void launch_embed_q8_0(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim,
                       hipStream_t s);
void launch_quant_q8_0(const float* x, uint8_t* y, int64_t n_elements, hipStream_t s);
void launch_q8_0_dispatch_T(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                            hipStream_t s);
void launch_q8_pad64(const float* x, uint8_t* out, int N, int K, hipStream_t s);
void launch_q8_pad64_dispatch_T(const uint8_t* Wp, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                                hipStream_t s);

// nan_mode: which reference form's NaN bits the NaN cells take: 0 = the scalar
// tiles of the dispatcher, 1 = bpd_qdot_q8_0_q8_0_cpu (the scalar build's llamafile).
void launch_q8_0_gemm_S(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                        int nan_mode, hipStream_t s);
// Up to 3 matrices of M[i] >= 1 rows sharing the activation rows Xq, one launch.
void launch_q8_0_gemm_S_multi(const uint8_t* const* W, float* const* out, const int* M, int n, const uint8_t* Xq,
                              int m_tokens, int K, int nan_mode, hipStream_t s);
// Gate and up (F rows each) with SwiGLU and its Q8_0 rows (yq, apart from Xq) in
// the epilogue; false (nothing launched) when the shape does not fit.
bool launch_q8_0_gemm_S_swiglu(const uint8_t* Wg, const uint8_t* Wu, int F, const uint8_t* Xq, int m_tokens, int K,
                               int nan_mode, uint8_t* yq, hipStream_t s);
void launch_stream_read(const uint8_t* p, int64_t n16, uint32_t* sink, hipStream_t s);
void launch_stream_write(uint8_t* p, int64_t n16, uint32_t value, hipStream_t s);
void launch_mfma_i8_probe(int waves, int iters, uint32_t* sink, hipStream_t s);

// Writes +0.0 to out[0..n).
void launch_fill_zero(float* out, int64_t n, hipStream_t s);
// bpd_qmm_q4k's cells: C[M][N] = deq(A[M][K]) . B[K][N], the reference's chain per cell.
void launch_qmm_q4k(const uint8_t* A, const float* B, float* C, int M, int N, int K, hipStream_t s);
// The AVX1 pair order P of bpd_qdot_q8_0_q8_0_cpu for every (activation row m, weight
// row n): out[m * n_rows + n]; Q8_0 rows of K/32 blocks (K <= qdot_p_max_k()).
int qdot_p_max_k();
void launch_q8_0_qdot_P(const uint8_t* Wq, const uint8_t* Xq, float* out, int n_rows, int m_tokens, int K,
                        hipStream_t s);

}  // namespace bpdq
