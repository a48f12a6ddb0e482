/* bpdq_oracle.h — CPU restatement of the reference quantized path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load liboracle.so, and only as the checker
 * or the timed CPU baseline.  The product path (libbpdq_hip.so) never calls it.
 *
 * Citations are /root/reference/<file>:<line>.
 */
#ifndef BPDQ_ORACLE_H
#define BPDQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* binary16 decode, three reference variants (identical on finite inputs). */
float bpdq_o_f16_ldexp(uint16_t h);   /* bench/bpd_quant.c:25-38 (NaN -> +/-0x7FC00000) */
float bpdq_o_f16_magic(uint16_t h);   /* bench/bpd_cpu.c:3928-3958 (NaN payload kept) */
float bpdq_o_f16_h2h(uint16_t h);     /* bench/bench_dequant_gpu_h2h.cu:14-19 (NaN -> +/-Inf) */
uint16_t bpdq_o_f32_to_f16(float f);  /* bench/bpd_cpu.c:4049-4104 */

/* Q4_K (144 B / 256 elements) */
void bpdq_o_dequant_q4k(const uint8_t* q, float* out, int n_blocks);       /* bench/bpd_quant.c:41-81 */
void bpdq_o_dequant_q4k_gguf(const uint8_t* q, float* out, int n_blocks);  /* bench/bench_dequant_gpu_h2h.cu:27-48 */
void bpdq_o_qmatmul_q4k(const uint8_t* w, const float* x, float* y, int M, int K);            /* bench/bpd_quant.c:88-109 */
void bpdq_o_qmm_q4k(const uint8_t* A, const float* B, float* C, int M, int N, int K);          /* bench/bpd_quant.c:114-137 */

/* Q8_K (292 B / 256 elements: f32 d, i8 qs[256], i16 bsums[16]) — no reference code exists. */
void bpdq_o_quant_q8_k(const float* x, uint8_t* y, int n);
/* y[r] = sum of Q4_K row r times Q8_K x; order 0 = bpd element map, 1 = GGUF element map. */
void bpdq_o_qmatmul_q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order);
/* exact per-super-block integer sums for one (row, block): I = sum sc_j S_j, Mn = sum m_j bsum_j */
void bpdq_o_q4k_q8k_block_ints(const uint8_t* wblk, const uint8_t* xblk, int order, int32_t* I, int32_t* Mn);

/* Q8_0 (34 B / 32 elements) */
/* Q6_K (210 B / 256): order 0 = inference/llamatov_helpers.py:161-179, order 1 = GGUF (llama.cpp) */
void bpdq_o_q6k_quants(const uint8_t* blk, int order, int8_t* q);
void bpdq_o_dequant_q6k(const uint8_t* q, float* out, int n_blocks, int order);
int32_t bpdq_o_q6k_q8k_block_int(const uint8_t* wblk, const uint8_t* xblk, int order);
void bpdq_o_qmatmul_q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order);

void bpdq_o_q8_pad64(const float* x, uint8_t* out, int N, int K);   /* inference/llamatov_c_inference.py:88-100 */

/* the reference Python loader's per-type fp32 dequant (inference/llamatov_helpers.py:196-222):
 * binary16 as numpy's astype, numpy float32 arithmetic in the expressions' order, x86 NaN bits */
float bpdq_o_f16_numpy(uint16_t h);
void bpdq_o_dequant_f16(const uint16_t* h, float* out, int64_t n);             /* :205-207 */
void bpdq_o_dequant_q4_0(const uint8_t* q, float* out, int n_blocks);          /* :71-98 */
void bpdq_o_dequant_q2k_py(const uint8_t* q, float* out, int n_blocks);        /* :25-39 */
void bpdq_o_dequant_q3k_py(const uint8_t* q, float* out, int n_blocks);        /* :42-68 */
void bpdq_o_dequant_q4k_py(const uint8_t* q, float* out, int n_blocks);        /* :101-158 */

void bpdq_o_dequant_q8_0(const uint8_t* raw, float* out, int n_blocks);                      /* bench/bpd_cpu.c:3960-3973 */
void bpdq_o_embed_lookup_q8_0(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim); /* :4002-4013 */
void bpdq_o_quant_q8_0(const float* x, uint8_t* y, int n_elements);                        /* bench/bpd_cpu.c:4106-4136 */
float bpdq_o_qdot_q8_0_S(const uint8_t* w, const uint8_t* a, int n_blocks);                 /* bench/bpd_cpu.c:4263-4280 */
float bpdq_o_qdot_q8_0_P(const uint8_t* w, const uint8_t* a, int n_blocks);                 /* bench/bpd_cpu.c:4208-4259 */
float bpdq_o_cell_q8_0_T(const uint8_t* w, const uint8_t* a, int n_blocks);                 /* bench/bpd_gemm_q8_0_cpu.c:32-86 */
float bpdq_o_cell_q8_0_S(const uint8_t* w, const uint8_t* a, int n_blocks);                 /* bench/bpd_gemm_q8_0_cpu.c:102-131 */
/* order: 'T' (AVX1 build tiles) or 'S' (scalar build tiles); out[token * m_weight + row]. */
void bpdq_o_dispatch_q8_0(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K, int order); /* bench/bpd_gemm_q8_0_cpu.c:159-207 */
/* order: 'P' (AVX1 qdot) or 'S'; out[m * N + n]. */
void bpdq_o_qmatmul_q8_0(const uint8_t* W, const float* X, float* out, int M, int N, int K, int order); /* bench/bpd_cpu.c:4295-4315 */
/* order: 'T' (AVX1 build) or 'S' (scalar build redirect, bench/bpd_cpu.c:4455-4458). */
void bpdq_o_qmatmul_q8_0_llamafile(const uint8_t* W, const float* X, float* out, int m_weight, int m_tokens, int K, int order); /* :4429-4452 */

/* ---- the decode step (bench/bpd_cpu.c:5611-5798) ---- */
/* expf by glibc's method (ARM optimized-routines expf, FMA variant); the table it uses. */
float bpdq_o_expf_nagy(float x);
void bpdq_o_expf_table(uint64_t* out32);
/* Inputs u = k*stride (k >= 0, u < 2^32, not NaN) where bpdq_o_expf_nagy and libm's expf differ. */
uint64_t bpdq_o_expf_mismatches(int nthreads, uint32_t stride, uint32_t* first_bad);
void bpdq_o_libm_expf(const float* x, float* y, int n);
void bpdq_o_rmsnorm(const float* x, const float* w, float* y, int n, float eps);           /* :4959-4986 */
void bpdq_o_rope_norm(float* t, int n_heads, int head_dim, int pos, float base);          /* :5146-5184 */
void bpdq_o_gqa_attn(const float* q, const float* kc, const float* vc, float* out, int max_seq, int pos, int H,
                     int HKV, int D, float scale);                                        /* :5370-5440 */
void bpdq_o_swiglu(const float* g, const float* u, float* y, int n);                      /* :5504-5507 */
int bpdq_o_argmax(const float* x, int n);                                                 /* :4512-4526 */
void bpdq_o_gemv_f32_wave(const float* W, const float* x, float* y, int N, int K);
typedef struct {
    const float* attn_norm;
    const uint8_t *q, *k, *v, *o;
    const float* ffn_norm;
    const uint8_t *gate, *up, *down;
    const float *q_bias, *k_bias, *v_bias;
} bpdq_o_layer;
typedef struct {
    int n_layers, n_embd, n_head, n_head_kv, head_dim, ff_dim, max_seq;
    float eps, rope_theta;
} bpdq_o_cfg;
/* fmt 0: Q8_0 rows, tile order T; 1 / 2: Q4_K (bpd / GGUF map) x Q8_K.  lm NULL: lm_f32 head. */
int bpdq_o_llama_step(int fmt, const bpdq_o_layer* layers, const bpdq_o_cfg* cfg, float* const* k_cache,
                      float* const* v_cache, int pos, const float* emb, const float* out_norm, const uint8_t* lm,
                      const float* lm_f32, int lm_N, float* x, float* h, float* logits);

/* bpd_rope_norm_freqs_cpu (bench/bpd_cpu.c:5146-5184) for one token: the first n_dims
 * elements of each head rotate in pairs, pair j by pos * theta_scale^j / freqs[j]
 * (freqs NULL: factor 1); the rest pass through. */
void bpdq_o_rope_norm_freqs(float* t, int n_heads, int head_dim, int pos, float base, int n_dims,
                            const float* freqs);
/* The step with per-matrix formats (fmts [n_layers][7] for q k v o gate up down, lm_fmt
 * for the head: 0 Q8_0 rows in tile order T, 1 / 2 Q4_K, 3 / 4 Q6_K in the bpd / GGUF
 * map, each K-quant against the Q8_K of its activation), rope_dim and frequency
 * factors (bpd_rope_norm_freqs_cpu), and binary16 caches (kv_f16: the caches are
 * uint16 arrays written with f32_to_f16 and read back with the magic-number
 * f16_to_f32, as bench/bpd_cpu.c:5659-5695 does). */
typedef struct {
    const int* fmts;
    int lm_fmt;
    int rope_dim;
    const float* rope_freqs;
    int kv_f16;
} bpdq_o_step_opts;
int bpdq_o_llama_step_ext(const bpdq_o_step_opts* o, const bpdq_o_layer* layers, const bpdq_o_cfg* cfg,
                          void* const* k_cache, void* const* v_cache, int pos, const float* emb,
                          const float* out_norm, const uint8_t* lm, const float* lm_f32, int lm_N, float* x,
                          float* h, float* logits);

/* Row-range parallel wrappers for the CPU baseline: every row's bits are those of
 * the single-threaded function. */
void bpdq_o_dequant_q4k_mt(const uint8_t* q, float* out, int n_blocks, int nthreads);
void bpdq_o_qmatmul_q4k_q8k_mt(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, int nthreads);
void bpdq_o_qmatmul_q6k_q8k_mt(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, int nthreads);
void bpdq_o_dispatch_q8_0_mt(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K, int order, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
