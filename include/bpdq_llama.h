/* bpdq_llama.h — the decode step of a llama-family model, part of
 * libbpdq_hip.so (gfx950 / MI355X).
 *
 * The structs and generate_token() are the ABI the reference's GPU driver binds
 * with ctypes (inference/llamatov_c_inference.py:15-83); the reference ships no
 * source for the library behind it.  What one step computes is the reference's
 * CPU transformer block, bpd_llama_block_cpu (bench/bpd_cpu.c:5611-5737), and the
 * head of bpd_llama_forward_cpu (:5740-5798), for one token at `position`:
 *
 *   per layer: h = rmsnorm(x) * attn_norm            (bpd_rmsnorm_llama_cpu, :4959)
 *              q, k, v = Wq h, Wk h, Wv h (+ bias)    (Q8_0 activations, tile order T)
 *              q, k = rope_norm(q, k, position)       (bpd_rope_norm_freqs_cpu, :5146)
 *              K/V cache[position] = k, v             (bpd_kv_cache_write_cpu, :5204)
 *              a = softmax(q k^T / sqrt(D)) v          (bpd_gqa_attn_cpu, :5370)
 *              x = x + Wo a
 *              h = rmsnorm(x) * ffn_norm
 *              x = x + Wdown (silu(Wgate h) * Wup h)  (bpd_swiglu_fuse_cpu, :5504)
 *   then       logits = W_lm (rmsnorm(x) * out_norm),  token = argmax (:4512)
 *
 * With Q8_0 weights in the padded layout, every fp32 operation happens in the
 * reference's order, including libm's expf, cosf and sinf, so logits and the
 * token are bit-identical to the reference's CPU block built for AVX (whose
 * Q8_0 product is the llamafile tile order).  Conditions: head_dim a multiple
 * of 32 and at most 256, n_head a multiple of n_head_kv, n_embd = n_head *
 * head_dim, every K a multiple of 32 (256 for Q4_K), n_embd <= 16384, and
 * K/V cache rows [0, position) written by earlier steps and finite.
 *
 * Differences from the reference's block, by design:
 *   - attention reads cache rows 0..position only; the reference scores all
 *     max_seq rows and masks the rest to weight 0, which adds exact zeros when
 *     those rows hold finite values;
 *   - RoPE has no frequency factors (the ABI carries none) and rope_dim = head_dim;
 *   - q/k/v biases (the qwen2 fields) are added to the projection before RoPE,
 *     as in llama.cpp's qwen2 graph; the reference block has no biases.
 * Calls run on the stream of bpd_gpu_set_stream() (include/bpdq.h); errors are
 * recorded for bpd_gpu_last_error().  The quantized activations and attention
 * scores live in the library's workspace of (device, stream): steps on one
 * stream run in order over it, steps on different streams use different
 * buffers.  It grows only outside stream capture (a step that would need it to
 * grow during capture fails with BPDQ_ERR_CAPTURE: run one step on that stream
 * first), and buffers it outgrows stay allocated for graphs captured with them
 * until bpd_gpu_workspace_release().
 */
#ifndef BPDQ_LLAMA_H
#define BPDQ_LLAMA_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* inference/llamatov_c_inference.py:15-31.  Weight pointers are device
 * pointers.  X_K is the input width (reduction length) and X_N the number of
 * output rows of matrix X: y[X_N] = W_X[X_N, X_K] h[X_K]. */
typedef struct {
    void* attn_norm; /* fp32 [n_embd] */
    void* q;
    void* k;
    void* v;
    void* o;
    void* ffn_norm; /* fp32 [n_embd] */
    void* gate;
    void* up;
    void* down;
    int q_K, q_N, k_K, k_N, v_K, v_N, o_K, o_N;
    int gate_K, gate_N, up_K, up_N, down_K, down_N;
    void* q_bias; /* fp32 [q_N] or NULL */
    void* k_bias; /* fp32 [k_N] or NULL */
    void* v_bias; /* fp32 [v_N] or NULL */
} LayerWeights;

/* :33-43 */
typedef struct {
    int n_layers, n_embd, n_head, n_head_kv, head_dim, ff_dim, vocab_size, max_seq;
    float eps, rope_theta;
} ModelConfig;

/* :45-51: two host arrays of n_layers device pointers, each to an fp32
 * [max_seq][n_head_kv * head_dim] cache. */
typedef struct {
    void** k_cache;
    void** v_cache;
} KVCache;

/* :53-59: device buffers, fp32 unless noted: x, h, q, attn_out, ffn [n_embd];
 * k, v [n_head_kv * head_dim]; gate, up [ff_dim]; logits [lm_N];
 * argmax_result: one int32.  After a step, x holds the residual stream after
 * the last layer, h the final normed x, logits the head's output. */
typedef struct {
    void* x;
    void* h;
    void* q;
    void* k;
    void* v;
    void* attn_out;
    void* gate;
    void* up;
    void* ffn;
    void* logits;
    void* argmax_result;
} WorkBuffers;

/* :62-78.  One decode step.  `embedding` is the fp32 [n_embd] input row on the
 * device (16-byte aligned, as are the norm weights, the work buffers and the
 * caches); layer and head weights are in the padded Q8 layout of
 * bpd_q8_pad64_from_f32_gpu (records [K/32][N][64]), or, with lm_head NULL,
 * the head is lm_f32: fp32 [lm_N][lm_K] row-major.  Returns the argmax token
 * (waits for the step to finish), or -1 after recording an error. */
int generate_token(const LayerWeights* layers, const ModelConfig* cfg, const WorkBuffers* buf, const KVCache* kv,
                   int position, const void* embedding, const void* output_norm_w, const void* lm_head,
                   const void* lm_f32, int lm_K, int lm_N);

/* :79-83.  gpu_alloc returns NULL on failure; copies are synchronous. */
void* gpu_alloc(int bytes);
void gpu_copy_h2d(void* dst_dev, const void* src_host, int bytes);
void gpu_copy_d2h(void* dst_host, const void* src_dev, int bytes);
void gpu_sync(void);
/* No counterpart in the reference (its driver never frees). */
void gpu_free(void* p);

/* ---- the same step for other weight formats, enqueued without waiting ----
 * No counterpart in the reference.  weight_format applies to the seven layer
 * matrices and lm_head:
 *   BPDQ_W_Q8_PAD64   the padded Q8 layout above (generate_token's format);
 *   BPDQ_W_Q4K        Q4_K GGUF bytes [N][K/256][144], bpd element map;
 *   BPDQ_W_Q4K_GGUF   Q4_K, GGUF (llama.cpp) element map.
 * With Q4_K weights each GEMV is the Q4_K x Q8_K product with the activation
 * quantized to Q8_K inside the kernel (bpd_qmatmul_q4k_q8k_fused_multi_gpu);
 * Q/K/V is one launch, and gate/up one launch that applies SwiGLU to its own
 * outputs (gate holds silu(gate) * up afterwards; up is not written).  The
 * token is left in
 * buf->argmax_result; returns 0, or -1 after recording an error.  For HIP
 * graph capture and timing loops. */
#define BPDQ_W_Q8_PAD64 0
#define BPDQ_W_Q4K 1
#define BPDQ_W_Q4K_GGUF 2
#define BPDQ_W_Q6K 3      /* Q6_K GGUF bytes [N][K/256][210], the reference's element map */
#define BPDQ_W_Q6K_GGUF 4 /* Q6_K, GGUF (llama.cpp) element map */
int bpd_llama_step_gpu(int weight_format, const LayerWeights* layers, const ModelConfig* cfg,
                       const WorkBuffers* buf, const KVCache* kv, int position, const void* embedding,
                       const void* output_norm_w, const void* lm_head, const void* lm_f32, int lm_K, int lm_N);

/* No counterpart in the reference's GPU ABI, whose ModelConfig has no room for
 * them; the reference's CPU block has each (bench/bpd_cpu.c:5556-5604).  The
 * same step with:
 *   layer_formats  host [n_layers][7] formats of q, k, v, o, gate, up, down
 *                  (NULL: weight_format everywhere).  A Q4_K_M file mixes
 *                  Q6_K into attn_v and ffn_down (inference/llamatov_helpers.py
 *                  dispatches per tensor type, :195-222).  Either every
 *                  matrix is BPDQ_W_Q8_PAD64 or none is (the K-quants take
 *                  Q8_K activations, the padded layout Q8_0 ones);
 *   lm_format      format of lm_head (-1: weight_format);
 *   rope_dim       elements of each head that rotate (0: head_dim), the
 *                  reference's cfg->rope_dim;
 *   rope_freqs     host [rope_dim / 2] frequency factors (Llama 3's
 *                  rope_freqs.weight) or NULL, read during the call;
 *   kv_cache_f16   1: the caches hold binary16 [max_seq][n_head_kv * head_dim]
 *                  (cfg->kv_cache_f16 of the reference; its f32_to_f16 bits on
 *                  write, f16_to_f32 on read).
 * A Q6_K gate/up pair, or one of two element maps, runs as two GEMVs and
 * SwiGLU; a Q6_K matrix reads the Q8_K of its activation. */
typedef struct {
    const int* layer_formats;
    int lm_format;
    int rope_dim;
    const float* rope_freqs;
    int kv_cache_f16;
} bpd_llama_step_opts;
int bpd_llama_step_ext_gpu(int weight_format, const bpd_llama_step_opts* opts, const LayerWeights* layers,
                           const ModelConfig* cfg, const WorkBuffers* buf, const KVCache* kv, int position,
                           const void* embedding, const void* output_norm_w, const void* lm_head, const void* lm_f32,
                           int lm_K, int lm_N);

/* ---- the reference's CPU transformer ABI, on the GPU ----
 * The structs and entry points of bench/bpd_cpu.c:5556-5798, argument for
 * argument, for n_tokens >= 1 (prefill, or one token at a time):
 * bpd_llama_block_gpu replaces bpd_llama_block_cpu (:5608-5737) and
 * bpd_llama_forward_gpu replaces bpd_llama_forward_cpu (:5740-5798).  Weights
 * are Q8_0 rows [N][K/32][34] (GGUF bytes unchanged); the caches are
 * [max_seq_len][n_kv_heads * head_dim] per layer, binary16 when
 * cfg->kv_cache_f16 (the reference's f32_to_f16 / f16_to_f32 bits) and fp32
 * otherwise.  RoPE follows bpd_rope_norm_freqs_cpu (:5146-5184): the first
 * rope_dim elements of each head rotate in pairs, pair j by pos_ids[t] *
 * theta_scale^j / rope_freqs[j], the rest pass through.
 *
 * Memory: every tensor is a device pointer (fp32 ones 16-byte aligned);
 * the structs, the layers array, token_ids, pos_ids and rope_freqs are host
 * memory, read before the call returns (the rotation angles are taken with
 * the host's libm, as the reference's cosf/sinf).  scratch1..3 hold at least
 * n_tokens * max(embed_dim, ffn_dim) floats each, as in the reference; they are
 * work space, and their contents after the call are not the reference's (the
 * _s_ forms form SwiGLU inside the gate/up GEMM and never write the gate, up or
 * SwiGLU rows).
 * token_out is int64 (the reference's long).  The calls enqueue on the
 * stream of bpd_gpu_set_stream() after one synchronization for the upload
 * of token ids, positions and angles; results are ready when that stream is.
 *
 * Order: bpd_llama_block_gpu / bpd_llama_forward_gpu give the bits of the
 * reference built with -mavx -mssse3 (its correctness build: Q8_0 products in
 * the llamafile tile order); the _s_ forms give those of its -O2 scalar build
 * (qdot order S, run on int8 MFMA).  Every other operation is shared.
 * Conditions: head_dim a multiple of 32, at most 256; embed_dim = n_heads *
 * head_dim, at most 16384; ffn_dim a multiple of 32; n_heads a multiple of
 * n_kv_heads; rope_dim even, 2 <= rope_dim <= head_dim; max_seq_len <= 32768;
 * kv_pos >= 0, kv_pos + n_tokens <= max_seq_len; every pos_ids[t] in
 * [0, max_seq_len); finite activations and cache contents.
 * Differences from the reference, by design:
 *   - attention reads cache rows 0..kv_pos+t for query t; the reference
 *     scores all max_seq_len rows and masks the rest to weight 0, which adds
 *     exact zeros when those rows hold finite values;
 *   - with fp32 caches, bpd_llama_forward_cpu steps from one layer's cache to
 *     the next by max_seq_len * n_kv_heads * head_dim uint16_t (:5771-5773),
 *     half an fp32 layer, so its layers overlap; bpd_llama_forward_gpu gives
 *     each layer a whole fp32 layer (the same bits while positions stay below
 *     max_seq_len / 2).  With binary16 caches (the reference driver's default,
 *     bench/bpd_llamatov_infer.py:453) the layouts are the same. */
typedef struct { /* bench/bpd_cpu.c:5556-5570 */
    int n_layers, n_heads, n_kv_heads, head_dim, embed_dim, ffn_dim, vocab_size, max_seq_len;
    float rms_eps, rope_base;
    int rope_dim, kv_cache_f16;
} bpd_llama_config;

typedef struct { /* :5585-5595, Q8_0 device tensors */
    const float* attn_norm_w;
    const uint8_t *w_q, *w_k, *w_v, *w_o;
    const float* ffn_norm_w;
    const uint8_t *w_gate, *w_up, *w_down;
} bpd_llama_layer_weights;

typedef struct { /* :5598-5604 */
    const uint8_t* token_embd;               /* Q8_0 [vocab_size][embed_dim] */
    const bpd_llama_layer_weights* layers;   /* host array of n_layers */
    const float* output_norm_w;              /* [embed_dim] */
    const uint8_t* output_w;                 /* Q8_0 [vocab_size][embed_dim] */
    const float* rope_freqs;                 /* host [rope_dim / 2], or NULL */
} bpd_llama_weights;

/* x: [n_tokens][embed_dim] in/out; k_cache, v_cache: this layer's caches. */
void bpd_llama_block_gpu(float* x, const bpd_llama_layer_weights* lw, const bpd_llama_config* cfg,
                         const int32_t* pos_ids, int n_tokens, int kv_pos, uint16_t* k_cache, uint16_t* v_cache,
                         float* scratch1, float* scratch2, float* scratch3, const float* rope_freqs);
void bpd_llama_block_s_gpu(float* x, const bpd_llama_layer_weights* lw, const bpd_llama_config* cfg,
                           const int32_t* pos_ids, int n_tokens, int kv_pos, uint16_t* k_cache, uint16_t* v_cache,
                           float* scratch1, float* scratch2, float* scratch3, const float* rope_freqs);
/* k_cache, v_cache: n_layers caches back to back; logits_out [n_tokens][vocab_size];
 * token_out [n_tokens] (the argmax of each row, bpd_argmax_dim_cpu). */
void bpd_llama_forward_gpu(const int32_t* token_ids, int n_tokens, const bpd_llama_weights* weights,
                           const bpd_llama_config* cfg, const int32_t* pos_ids, int kv_pos, uint16_t* k_cache,
                           uint16_t* v_cache, float* logits_out, int64_t* token_out);
void bpd_llama_forward_s_gpu(const int32_t* token_ids, int n_tokens, const bpd_llama_weights* weights,
                             const bpd_llama_config* cfg, const int32_t* pos_ids, int kv_pos, uint16_t* k_cache,
                             uint16_t* v_cache, float* logits_out, int64_t* token_out);

/* ---- single steps of the decode step, for parity tests ----
 * x_out = x_in (+ add); h = rmsnorm(x_out) * w; xq = Q8_0(h) when xq != NULL
 * (bpd_rmsnorm_llama_cpu, bench/bpd_cpu.c:4959-4986, with the residual add of
 * bpd_add_f32_cpu, :5466, in front).  The sum of squares is accumulated in
 * binary64 as the reference does; when the parallel sum cannot prove that the
 * reference's sequential binary64 sum rounds to the same fp32 mean, the kernel
 * recomputes it sequentially.  fp32 pointers 16-byte aligned. */
void bpd_residual_rmsnorm_gpu(const float* x_in, const float* add, float* x_out, const float* w, float* h,
                              uint8_t* xq, int n, float eps);
/* out[0] = the step's argmax of x[n] (bpd_argmax_dim_cpu, bench/bpd_cpu.c:4512-4526,
 * with outer = inner = 1): first index of the largest non-NaN value, 0 when x[0]
 * is NaN.  x 16-byte aligned. */
void bpd_argmax_gpu(const float* x, int n, int32_t* out);
/* expf of the decode step (the platform libm's, see bpdq_math.h) on n values. */
void bpd_expf_gpu(const float* x, float* y, int n);

#ifdef __cplusplus
}
#endif
#endif
