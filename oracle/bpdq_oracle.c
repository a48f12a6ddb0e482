/* bpdq_oracle.c — CPU restatement of the reference Q4_K / Q8_0 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker the HIP kernels are compared
 * against, and the CPU baseline bench.py times.  Nothing in the product library
 * links or calls it.  Build with gcc -O2 -ffp-contract=off (no -march, no
 * -ffast-math): every fp32 operation below is one IEEE binary32 operation
 * rounded to nearest even, in the order written.
 *
 * Each function cites the reference code (/root/reference/<file>:<line>) whose
 * operation order it restates.  The Q8_K quantizer and the Q4_K x Q8_K dot have
 * no reference code (the reference lists Q8_K only by size,
 * lib/gguf_emit_manifest.pl:130,142); their order is defined here and shared
 * with the GPU kernel:
 *
 *   per super-block b of a row (256 elements, sub-blocks j = 0..7):
 *     S_j  = sum over the 32 elements of sub-block j of q4 * q8   (exact int)
 *     I_b  = sum_j sc_j * S_j                                       (exact int32)
 *     Mn_b = sum_j m_j * (bsums[2j] + bsums[2j+1])                  (exact int32)
 *     c_b  = RN( RN(RN(d*dy) * float(I_b)) - RN(RN(dmin*dy) * float(Mn_b)) )
 *   per row, with nb super-blocks:
 *     s_q  = +0.0;  for b = q, q+8, q+16, ... < nb:  s_q = RN(s_q + c_b)   (q = 0..7)
 *     y    = RN( RN(RN(s0+s1) + RN(s2+s3)) + RN(RN(s4+s5) + RN(s6+s7)) )
 */
#include "bpdq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 ---- */

/* bench/bpd_quant.c:25-38 (same arithmetic: bench/bpd_quant_gpu.cu:19-30,
 * bench/bpd_gemm_q8_0_cpu.c:13-26).  mant/1024 and the ldexpf scaling are exact,
 * so every finite input decodes to its exact value; NaN decodes to +/-NAN. */
float bpdq_o_f16_ldexp(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    float r;
    if (e == 0) r = m ? ldexpf((float)m, -24) : 0.0f;
    else if (e == 31) r = m ? NAN : INFINITY;
    else r = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -r : r;
}

/* bench/bpd_cpu.c:3928-3958.  The magic-number form yields the exact value for
 * finite inputs and, for NaN, the f16 payload shifted up with the quiet bit set
 * (the multiply by 2^-112 quiets a signalling NaN). */
float bpdq_o_f16_magic(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u, bits;
    if (e == 31) {
        bits = s | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u);
    } else {
        float v = e ? ldexpf((float)(m | 1024u), (int)e - 25) : ldexpf((float)m, -24);
        memcpy(&bits, &v, 4);
        bits |= s;
    }
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* bench/bench_dequant_gpu_h2h.cu:14-19: +/-0 both decode to +0.0, NaN decodes
 * to +/-Inf, everything else exactly. */
float bpdq_o_f16_h2h(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0 && m == 0) return 0.0f;
    if (e == 31) return s ? -INFINITY : INFINITY;
    float v = e ? ldexpf((float)(m | 1024u), (int)e - 25) : ldexpf((float)m, -24);
    return s ? -v : v;
}

/* bench/bpd_cpu.c:4049-4104: binary32 -> binary16, round to nearest even,
 * overflow -> Inf, NaN -> exponent 31 with the top mantissa bits and bit 0 set. */
uint16_t bpdq_o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ef = (x >> 23) & 0xFFu, mf = x & 0x7FFFFFu;
    if (ef == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mf ? ((mf >> 13) | 1u) : 0u));
    int32_t eh = (int32_t)ef - 112;
    if (eh >= 31) return (uint16_t)(sign | 0x7C00u);
    if (eh <= 0) {
        if (eh < -10) return (uint16_t)sign;
        uint32_t full = mf | 0x800000u;
        int sh = 14 - eh;
        uint32_t q = full >> sh;
        uint32_t rb = (full >> (sh - 1)) & 1u;
        uint32_t st = (full & ((1u << (sh - 1)) - 1u)) != 0u;
        if (rb && (st || (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = mf >> 13;
    uint32_t rb = (mf >> 12) & 1u, st = (mf & 0xFFFu) != 0u;
    if (rb && (st || (q & 1u))) {
        q++;
        if (q == 0x400u) {
            q = 0;
            eh++;
            if (eh >= 31) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)eh << 10) | q);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* (int8_t)v for a float v, as the reference's x86 build executes the cast of
 * bench/bpd_cpu.c:4133 (also used for the Q8_K and padded-Q8 quantizers below):
 * cvttss2si to int32, which gives 0x80000000 for NaN and for values outside the
 * int32 range, then the low byte.  Spelled out because the C cast is undefined
 * for such v (a NaN element, or an overflowing 127/amax). */
static inline int8_t x86_f32_to_i8(float v) {
    const int32_t i = (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : INT32_MIN;  /* NaN: both false */
    return (int8_t)(uint8_t)(uint32_t)i;
}

/* ------------------------------------------------------- x86 NaN rules --- */

/* The reference's compiled C runs on x86, whose SSE arithmetic gives a NaN
 * operand back quieted (the first operand's when both are NaN) and the default
 * NaN 0xFFC00000 for an invalid operation (Inf*0, Inf-Inf).  For a product or
 * sum whose two operands can both be NaN, the output bits therefore depend on
 * which operand the compiler put first.  These helpers fix that choice in the
 * source; each call site names the operand the reference build puts first
 * (measured on oracle/_ref and pinned by tests/test_oracle_reference.py). */
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline float x86_nan_of(float a, float b) {
    if (isnan(a)) return bits_f32(f32_bits(a) | 0x400000u);
    if (isnan(b)) return bits_f32(f32_bits(b) | 0x400000u);
    return bits_f32(0xFFC00000u);
}
static inline float x86_mul(float first, float second) {
    float r = first * second;
    return isnan(r) ? x86_nan_of(first, second) : r;
}
static inline float x86_add(float first, float second) {
    float r = first + second;
    return isnan(r) ? x86_nan_of(first, second) : r;
}

/* ---------------------------------------------------------------- Q4_K --- */

/* 6-bit scale/min of sub-block j: bench/bpd_quant.c:56-62. */
static inline void q4k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* bench/bpd_quant.c:41-74: element 32j+k <- low nibble of qs[16j+k],
 * element 32j+16+k <- high nibble; y = RN(d*sc*q - dmin*m). */
static void dq_block_bpd(const uint8_t* blk, float* out) {
    float d = bpdq_o_f16_ldexp(rd16(blk)), dmin = bpdq_o_f16_ldexp(rd16(blk + 2));
    const uint8_t* s = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_scale_min(s, j, &sc, &m);
        float scale = d * (float)sc, mn = dmin * (float)m;
        for (int k = 0; k < 16; k++) {
            uint8_t byte = qs[16 * j + k];
            out[32 * j + k] = scale * (float)(byte & 15) - mn;
            out[32 * j + 16 + k] = scale * (float)(byte >> 4) - mn;
        }
    }
}

void bpdq_o_dequant_q4k(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) dq_block_bpd(q + (size_t)b * 144, out + (size_t)b * 256);
}

/* The GGUF-map dequant exists in the reference only as a CUDA kernel, so its
 * NaN outputs are the NVIDIA GPU's: every fp32 operation that yields a NaN
 * there returns the canonical NaN 0x7FFFFFFF (PTX ISA, floating-point
 * instructions: NaN payloads are not propagated). */
static inline float cuda_nan(float y) { return isnan(y) ? bits_f32(0x7FFFFFFFu) : y; }

/* bench/bench_dequant_gpu_h2h.cu:27-48: for i in 0..3, l in 0..31:
 * element 64i+l <- low(qs[32i+l]) with sub-block 2i,
 * element 64i+32+l <- high(qs[32i+l]) with sub-block 2i+1; h2h f16 decode. */
void bpdq_o_dequant_q4k_gguf(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 144;
        float* y = out + (size_t)b * 256;
        float dall = bpdq_o_f16_h2h(rd16(blk)), dmin = bpdq_o_f16_h2h(rd16(blk + 2));
        for (int i = 0; i < 4; i++) {
            int sc, m;
            q4k_scale_min(blk + 4, 2 * i, &sc, &m);
            float d1 = dall * (float)sc, m1 = dmin * (float)m;
            q4k_scale_min(blk + 4, 2 * i + 1, &sc, &m);
            float d2 = dall * (float)sc, m2 = dmin * (float)m;
            const uint8_t* qs = blk + 16 + 32 * i;
            for (int l = 0; l < 32; l++) {
                y[64 * i + l] = cuda_nan(d1 * (float)(qs[l] & 15) - m1);
                y[64 * i + 32 + l] = cuda_nan(d2 * (float)(qs[l] >> 4) - m2);
            }
        }
    }
}

/* bench/bpd_quant.c:88-109: sequential fp32 chain from +0.0 over k in element order. */
void bpdq_o_qmatmul_q4k(const uint8_t* w, const float* x, float* y, int M, int K) {
    int nb = K / 256;
    float buf[256];
    for (int r = 0; r < M; r++) {
        float sum = 0.0f;
        const uint8_t* row = w + (size_t)r * nb * 144;
        for (int b = 0; b < nb; b++) {
            dq_block_bpd(row + (size_t)b * 144, buf);
            const float* xp = x + (size_t)b * 256;
            /* the reference build multiplies with the weight first and adds onto sum */
            for (int k = 0; k < 256; k++) sum = x86_add(sum, x86_mul(buf[k], xp[k]));
        }
        y[r] = sum;
    }
}

/* bench/bpd_quant.c:114-137: C[r,c] = sequential chain over k of deq(A)[r,k]*B[k,c]. */
void bpdq_o_qmm_q4k(const uint8_t* A, const float* B, float* C, int M, int N, int K) {
    int nb = K / 256;
    float buf[256];
    for (int r = 0; r < M; r++) {
        const uint8_t* row = A + (size_t)r * nb * 144;
        for (int c = 0; c < N; c++) C[(size_t)r * N + c] = 0.0f;
        for (int b = 0; b < nb; b++) {
            dq_block_bpd(row + (size_t)b * 144, buf);
            for (int k = 0; k < 256; k++) {
                float a = buf[k];
                const float* brow = B + ((size_t)b * 256 + k) * N;
                /* the reference build puts B first in the product and the product first in the sum */
                for (int c = 0; c < N; c++) C[(size_t)r * N + c] = x86_add(x86_mul(brow[c], a), C[(size_t)r * N + c]);
            }
        }
    }
}

/* ---------------------------------------------------------------- Q8_K --- */

/* Q8_K quantizer (no reference code).  Mirrors the Q8_0 rule of
 * bench/bpd_cpu.c:4106-4136 at 256 elements with an fp32 scale:
 * d = RN(amax/127), id = amax ? RN(127/amax) : 0, q = rint(RN(x*id)),
 * bsums[g] = sum of q over elements 16g..16g+15. */
void bpdq_o_quant_q8_k(const float* x, uint8_t* y, int n) {
    int nb = n / 256;
    for (int b = 0; b < nb; b++) {
        const float* xb = x + (size_t)b * 256;
        uint8_t* yb = y + (size_t)b * 292;
        float amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            float v = xb[j];
            float av = v < 0 ? -v : v;
            if (av > amax) amax = av;
        }
        float d = amax / 127.0f;
        float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        memcpy(yb, &d, 4);
        int8_t* qs = (int8_t*)(yb + 4);
        for (int j = 0; j < 256; j++) qs[j] = x86_f32_to_i8(rintf(xb[j] * id));
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) s += qs[16 * g + j];
            int16_t s16 = (int16_t)s;
            memcpy(yb + 260 + 2 * g, &s16, 2);
        }
    }
}

void bpdq_o_q4k_q8k_block_ints(const uint8_t* wblk, const uint8_t* xblk, int order, int32_t* I, int32_t* Mn) {
    const uint8_t* s = wblk + 4;
    const uint8_t* qs = wblk + 16;
    const int8_t* xq = (const int8_t*)(xblk + 4);
    int32_t S[8] = {0};
    if (order == 0) {
        for (int j = 0; j < 8; j++)
            for (int k = 0; k < 16; k++)
                S[j] += (qs[16 * j + k] & 15) * xq[32 * j + k] + (qs[16 * j + k] >> 4) * xq[32 * j + 16 + k];
    } else {
        for (int i = 0; i < 4; i++)
            for (int l = 0; l < 32; l++) {
                S[2 * i] += (qs[32 * i + l] & 15) * xq[64 * i + l];
                S[2 * i + 1] += (qs[32 * i + l] >> 4) * xq[64 * i + 32 + l];
            }
    }
    int32_t isum = 0, msum = 0;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_scale_min(s, j, &sc, &m);
        int16_t b0, b1;
        memcpy(&b0, xblk + 260 + 4 * j, 2);
        memcpy(&b1, xblk + 262 + 4 * j, 2);
        isum += sc * S[j];
        msum += m * ((int32_t)b0 + (int32_t)b1);
    }
    *I = isum;
    *Mn = msum;
}

static float q4k_q8k_row(const uint8_t* row, const uint8_t* xq, int nb, int order) {
    float s[8];
    for (int q = 0; q < 8; q++) s[q] = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = row + (size_t)b * 144;
        const uint8_t* xb = xq + (size_t)b * 292;
        int32_t I, Mn;
        bpdq_o_q4k_q8k_block_ints(wb, xb, order, &I, &Mn);
        float dy;
        memcpy(&dy, xb, 4);
        float dd = bpdq_o_f16_magic(rd16(wb)) * dy;
        float dm = bpdq_o_f16_magic(rd16(wb + 2)) * dy;
        float a = dd * (float)I;
        float m = dm * (float)Mn;
        float c = a - m;
        s[b & 7] = s[b & 7] + c;
    }
    float t0 = s[0] + s[1], t1 = s[2] + s[3], t2 = s[4] + s[5], t3 = s[6] + s[7];
    return (t0 + t1) + (t2 + t3);
}

void bpdq_o_qmatmul_q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order) {
    int nb = K / 256;
    for (int r = 0; r < M; r++) y[r] = q4k_q8k_row(w + (size_t)r * nb * 144, xq, nb, order);
}

/* ---------------------------------------------------------------- Q6_K --- */

/* Q6_K block, 210 B per 256 elements: ql[128] (low 4 bits), qh[64] (high 2
 * bits), sc[16] (int8, one per 16 elements), d (f16 at byte 208).
 * q = (low | high << 4) - 32.  Element maps:
 *   order 0, inference/llamatov_helpers.py:161-179: element 2i takes the low
 *     nibble of ql[i], 2i+1 its high nibble; element 4j+k takes bits 2k..2k+1
 *     of qh[j];
 *   order 1, the GGUF layout of llama.cpp's dequantize_row_q6_K (ggml-quants.c,
 *     the llama.cpp build 5311 the reference audits, docs/llama-kernel-audit.md:11):
 *     in half h (ql += 64h, qh += 32h), for l < 32: element l takes ql[l] low and
 *     qh[l] bits 0-1, l+32 ql[l+32] low and bits 2-3, l+64 ql[l] high and bits
 *     4-5, l+96 ql[l+32] high and bits 6-7.
 * In both maps element e uses scale sc[e/16]. */
void bpdq_o_q6k_quants(const uint8_t* blk, int order, int8_t* q) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    if (order == 0) {
        for (int i = 0; i < 128; i++) {
            int e0 = 2 * i, e1 = 2 * i + 1;
            q[e0] = (int8_t)(((ql[i] & 15) | (((qh[e0 / 4] >> (2 * (e0 % 4))) & 3) << 4)) - 32);
            q[e1] = (int8_t)(((ql[i] >> 4) | (((qh[e1 / 4] >> (2 * (e1 % 4))) & 3) << 4)) - 32);
        }
    } else {
        for (int h = 0; h < 2; h++) {
            const uint8_t* L = ql + 64 * h;
            const uint8_t* H = qh + 32 * h;
            int8_t* o = q + 128 * h;
            for (int l = 0; l < 32; l++) {
                o[l] = (int8_t)(((L[l] & 15) | (((H[l] >> 0) & 3) << 4)) - 32);
                o[l + 32] = (int8_t)(((L[l + 32] & 15) | (((H[l] >> 2) & 3) << 4)) - 32);
                o[l + 64] = (int8_t)(((L[l] >> 4) | (((H[l] >> 4) & 3) << 4)) - 32);
                o[l + 96] = (int8_t)(((L[l + 32] >> 4) | (((H[l] >> 6) & 3) << 4)) - 32);
            }
        }
    }
}

/* y = (d * sc) * q in fp32: d*sc is exact (11 x 8 bits), so one rounding,
 * as the float32 numpy of inference/llamatov_helpers.py:177-178 and the C of
 * dequantize_row_q6_K.  The scale is decoded with NaN payloads kept. */
void bpdq_o_dequant_q6k(const uint8_t* q, float* out, int n_blocks, int order) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 210;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = bpdq_o_f16_magic(rd16(blk + 208));
        int8_t qq[256];
        bpdq_o_q6k_quants(blk, order, qq);
        for (int e = 0; e < 256; e++) {
            float ds = d * (float)sc[e / 16];
            out[(size_t)b * 256 + e] = ds * (float)qq[e];
        }
    }
}

/* ------------------------------------- the reference Python loader ---- */

/* load_tensor_by_type (inference/llamatov_helpers.py:196-222) turns each GGUF
 * tensor into fp32 with numpy float32 arithmetic: binary16 through astype (the
 * exact value; a NaN keeps its payload and its signalling bit), every product
 * and difference one float32 operation with the left operand of the Python
 * expression first, under x86's NaN rules (x86_mul / x86_sub).  Q6_K is
 * bpdq_o_dequant_q6k order 0. */
static inline float x86_sub(float first, float second) {
    float r = first - second;
    return isnan(r) ? x86_nan_of(first, second) : r;
}

/* numpy's float16 -> float32 (astype): sign, exponent 255 and the payload
 * shifted up for Inf / NaN, no quiet bit added; finite values exactly. */
float bpdq_o_f16_numpy(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return bits_f32(s | 0x7F800000u | (m << 13));
    float v = e ? ldexpf((float)(m | 1024u), (int)e - 25) : ldexpf((float)m, -24);
    return bits_f32(f32_bits(v) | s);
}

/* TYPE_F16 (:205-207). */
void bpdq_o_dequant_f16(const uint16_t* h, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = bpdq_o_f16_numpy(h[i]);
}

/* dequant_q4_0 (:71-98), 18-byte blocks {f16 d, u8 qs[16]}: element e < 16 is
 * the low nibble of qs[e], element 16 + e the high one; y = d * (q - 8.0). */
void bpdq_o_dequant_q4_0(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 18;
        const float d = bpdq_o_f16_numpy(rd16(blk));
        for (int e = 0; e < 32; e++) {
            const int v = e < 16 ? (blk[2 + e] & 15) : (blk[2 + e - 16] >> 4);
            out[(size_t)b * 32 + e] = x86_mul(d, (float)v - 8.0f);
        }
    }
}

/* The 2-bit field of element e (0..255) in the Python loader's unpack: bits
 * 2(e%4)..+1 of qs[e/4] (np.stack([(qs >> 2i) & 3], -1).reshape). */
static inline int py_q2(const uint8_t* qs, int e) { return (qs[e >> 2] >> (2 * (e & 3))) & 3; }

/* dequant_q2_k (:25-39), 84-byte blocks {u8 scales[16], u8 qs[64], f16 d, f16
 * dmin}: sc = (scales[i] & 15) * d, mn = (scales[i] >> 4) * dmin, y = sc * q - mn
 * with i = e / 16 and q the Python unpack's 2-bit field. */
void bpdq_o_dequant_q2k_py(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 84;
        const float d = bpdq_o_f16_numpy(rd16(blk + 80)), dm = bpdq_o_f16_numpy(rd16(blk + 82));
        for (int e = 0; e < 256; e++) {
            const int sb = blk[e / 16];
            const float sc = x86_mul((float)(sb & 15), d), mn = x86_mul((float)(sb >> 4), dm);
            out[(size_t)b * 256 + e] = x86_sub(x86_mul(sc, (float)py_q2(blk + 16, e)), mn);
        }
    }
}

/* dequant_q3_k (:42-68, the approximate form the reference itself marks as
 * such), 110-byte blocks {u8 hmask[32], u8 qs[64], u8 scales[12], f16 d}:
 * scale i < 8 = (scales[i] & 15) - 8, scale 8 + i = (scales[i] >> 4) - 8 (bytes
 * 8..11 unused); quant = q_lo + 4 * hbit - 4 with q_lo the 2-bit field and hbit
 * bit e%8 of hmask[e/8]; y = (d * scale[e/16]) * quant. */
void bpdq_o_dequant_q3k_py(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 110;
        const float d = bpdq_o_f16_numpy(rd16(blk + 108));
        for (int e = 0; e < 256; e++) {
            const int i = e / 16, sbyte = blk[96 + (i & 7)];
            const float scale = (float)(i < 8 ? (sbyte & 15) : (sbyte >> 4)) - 8.0f;
            const float quant = (float)py_q2(blk + 32, e) + (float)((blk[e >> 3] >> (e & 7)) & 1) * 4.0f - 4.0f;
            out[(size_t)b * 256 + e] = x86_mul(x86_mul(d, scale), quant);
        }
    }
}

/* dequant_q4_k (:101-158): the 6-bit scales and mins of bench/bpd_quant.c:56-62,
 * and the Python loader's own element map: element e < 128 is the low nibble
 * of qs[e] in sub-block e/32, element 128 + e the high nibble of qs[e] in
 * sub-block 4 + e/32; y = ((d * sc) * q) - (dmin * m). */
void bpdq_o_dequant_q4k_py(const uint8_t* q, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = q + (size_t)b * 144;
        const float d = bpdq_o_f16_numpy(rd16(blk)), dmin = bpdq_o_f16_numpy(rd16(blk + 2));
        for (int e = 0; e < 256; e++) {
            const int hi = e >= 128, i = e & 127, j = (hi ? 4 : 0) + i / 32;
            int sc, m;
            q4k_scale_min(blk + 4, j, &sc, &m);
            const int v = hi ? blk[16 + i] >> 4 : blk[16 + i] & 15;
            out[(size_t)b * 256 + e] = x86_sub(x86_mul(x86_mul(d, (float)sc), (float)v), x86_mul(dmin, (float)m));
        }
    }
}

/* Q6_K x Q8_K (no reference code; the reference dequantizes Q6_K to fp32 in
 * Python): I_b = sum over the 16 groups g of sc[g] * sum_{e in g} q_e * x_e,
 * exact in int32; c_b = RN(RN(d*dy) * float(I_b)); then the fixed fp32 order of
 * the Q4_K x Q8_K GEMV: slot sums s_q from +0.0 over b = q mod 8 ascending,
 * y = ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)). */
int32_t bpdq_o_q6k_q8k_block_int(const uint8_t* wblk, const uint8_t* xblk, int order) {
    int8_t qq[256];
    bpdq_o_q6k_quants(wblk, order, qq);
    const int8_t* sc = (const int8_t*)(wblk + 192);
    const int8_t* xq = (const int8_t*)(xblk + 4);
    int32_t I = 0;
    for (int g = 0; g < 16; g++) {
        int32_t S = 0;
        for (int k = 0; k < 16; k++) S += qq[16 * g + k] * xq[16 * g + k];
        I += sc[g] * S;
    }
    return I;
}

static float q6k_q8k_row(const uint8_t* row, const uint8_t* xq, int nb, int order) {
    float s[8];
    for (int q = 0; q < 8; q++) s[q] = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = row + (size_t)b * 210;
        const uint8_t* xb = xq + (size_t)b * 292;
        int32_t I = bpdq_o_q6k_q8k_block_int(wb, xb, order);
        float dy;
        memcpy(&dy, xb, 4);
        float dd = bpdq_o_f16_magic(rd16(wb + 208)) * dy;
        float c = dd * (float)I;
        s[b & 7] = s[b & 7] + c;
    }
    float t0 = s[0] + s[1], t1 = s[2] + s[3], t2 = s[4] + s[5], t3 = s[6] + s[7];
    return (t0 + t1) + (t2 + t3);
}

void bpdq_o_qmatmul_q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order) {
    int nb = K / 256;
    for (int r = 0; r < M; r++) y[r] = q6k_q8k_row(w + (size_t)r * nb * 210, xq, nb, order);
}

/* ---------------------------------------------------------------- Q8_0 --- */

/* bench/bpd_cpu.c:3960-3973 */
void bpdq_o_dequant_q8_0(const uint8_t* raw, float* out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const uint8_t* blk = raw + (size_t)b * 34;
        float d = bpdq_o_f16_magic(rd16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        for (int i = 0; i < 32; i++) out[(size_t)b * 32 + i] = (float)qs[i] * d;
    }
}

/* bench/bpd_cpu.c:4002-4013 */
void bpdq_o_embed_lookup_q8_0(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim) {
    int bpr = embed_dim / 32;
    for (int t = 0; t < n_tokens; t++)
        bpdq_o_dequant_q8_0(table + (size_t)ids[t] * bpr * 34, out + (size_t)t * embed_dim, bpr);
}

/* bench/bpd_cpu.c:4106-4136 */
void bpdq_o_quant_q8_0(const float* x, uint8_t* y, int n_elements) {
    int nb = n_elements / 32;
    for (int i = 0; i < nb; i++) {
        const float* xb = x + (size_t)i * 32;
        uint8_t* yb = y + (size_t)i * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = xb[j];
            float av = v < 0 ? -v : v;
            if (av > amax) amax = av;
        }
        uint16_t dh = bpdq_o_f32_to_f16(amax / 127.0f);
        yb[0] = (uint8_t)(dh & 0xFF);
        yb[1] = (uint8_t)(dh >> 8);
        float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        int8_t* qs = (int8_t*)(yb + 2);
        for (int j = 0; j < 32; j++) qs[j] = x86_f32_to_i8(rintf(xb[j] * id));
    }
}

/* SSSE3 _mm_sign_epi8 + _mm_maddubs_epi16 + _mm_madd_epi16(1) on four bytes,
 * with the weight byte as the sign source (bench/bpd_cpu.c:4166-4170,
 * bench/bpd_gemm_q8_0_cpu.c:58-66).  Equals the true dot product unless an
 * activation byte is -128 against a negative weight (the negation wraps). */
static inline int32_t sse_quad(const int8_t* w, const int8_t* a) {
    int32_t pair[2];
    for (int h = 0; h < 2; h++) {
        int32_t t = 0;
        for (int u = 0; u < 2; u++) {
            int wi = w[2 * h + u], ai = a[2 * h + u];
            int ua = wi < 0 ? -wi : wi;                                   /* |w|, 128 for -128 */
            int sb = wi < 0 ? (int)(int8_t)(uint8_t)(-ai) : (wi == 0 ? 0 : ai);
            t += ua * sb;
        }
        if (t > 32767) t = 32767;
        if (t < -32768) t = -32768;
        pair[h] = t;
    }
    return pair[0] + pair[1];
}

static inline float hsum8(const float* a) {
    /* bench/bpd_cpu.c:4200-4206 */
    return ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}

static inline int32_t dot32(const int8_t* w, const int8_t* a) {
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += (int32_t)w[j] * (int32_t)a[j];
    return s;
}

/* Scalar order S: bench/bpd_cpu.c:4263-4280 and bench/bpd_gemm_q8_0_cpu.c:112-128. */
float bpdq_o_qdot_q8_0_S(const uint8_t* w, const uint8_t* a, int n_blocks) {
    float sumf = 0.0f;
    for (int ib = 0; ib < n_blocks; ib++) {
        const uint8_t* wb = w + (size_t)ib * 34;
        const uint8_t* ab = a + (size_t)ib * 34;
        int32_t sumi = dot32((const int8_t*)(wb + 2), (const int8_t*)(ab + 2));
        /* the reference build puts the weight scale first */
        float delta = x86_mul(bpdq_o_f16_magic(rd16(wb)), bpdq_o_f16_magic(rd16(ab)));
        sumf = x86_add(sumf, (float)sumi * delta);
    }
    return sumf;
}

/* Scalar tile cell: bench/bpd_gemm_q8_0_cpu.c:112-128.  The same sum as
 * bpdq_o_qdot_q8_0_S, but its scales are decoded by the ldexpf form of
 * bench/bpd_gemm_q8_0_cpu.c:13-26 (NaN -> +/-0x7FC00000, no payload) and the
 * reference build puts the activation scale Bd first in Ad*Bd. */
float bpdq_o_cell_q8_0_S(const uint8_t* w, const uint8_t* a, int n_blocks) {
    float sumf = 0.0f;
    for (int l = 0; l < n_blocks; l++) {
        const uint8_t* wb = w + (size_t)l * 34;
        const uint8_t* ab = a + (size_t)l * 34;
        int32_t sumi = dot32((const int8_t*)(wb + 2), (const int8_t*)(ab + 2));
        float delta = x86_mul(bpdq_o_f16_ldexp(rd16(ab)), bpdq_o_f16_ldexp(rd16(wb)));
        sumf = x86_add(sumf, (float)sumi * delta);
    }
    return sumf;
}

/* AVX1 pair order P: bench/bpd_cpu.c:4208-4259. */
/* NaN bits as the reference build gives them (measured with probes of two NaNs of
 * different sign and payload per operand pair): the pair deltas put the activation
 * scale first, the lane chains the accumulator first (the first NaN of a lane
 * sticks), the odd block's delta the weight scale first and its add the running sum
 * first; the hsum's additions, with the left operand of
 * ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)) first unless noted, take a4 before a0, a5 before
 * a1, the (a2,a6) sum before the (a0,a4) one and the (a3,a7) sum before the (a1,a5)
 * one.  (Orders within the right half that no input can tell apart are not pinned:
 * its NaNs are always default NaNs when the left half holds none.) */
float bpdq_o_qdot_q8_0_P(const uint8_t* w, const uint8_t* a, int n_blocks) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int ib = 0;
    for (; ib + 1 < n_blocks; ib += 2) {
        for (int h = 0; h < 2; h++) {
            const uint8_t* wb = w + (size_t)(ib + h) * 34;
            const uint8_t* ab = a + (size_t)(ib + h) * 34;
            const int8_t* wq = (const int8_t*)(wb + 2);
            const int8_t* aq = (const int8_t*)(ab + 2);
            float delta = x86_mul(bpdq_o_f16_magic(rd16(ab)), bpdq_o_f16_magic(rd16(wb)));
            for (int i = 0; i < 4; i++) {
                int32_t p = sse_quad(wq + 4 * i, aq + 4 * i) + sse_quad(wq + 16 + 4 * i, aq + 16 + 4 * i);
                float prod = x86_mul(delta, (float)p);
                acc[4 * h + i] = x86_add(acc[4 * h + i], prod);
            }
        }
    }
    float l0 = x86_add(acc[4], acc[0]), l1 = x86_add(acc[2], acc[6]);
    float l2 = x86_add(acc[5], acc[1]), l3 = x86_add(acc[3], acc[7]);
    float sumf = x86_add(x86_add(l1, l0), x86_add(l3, l2));
    for (; ib < n_blocks; ib++) {
        const uint8_t* wb = w + (size_t)ib * 34;
        const uint8_t* ab = a + (size_t)ib * 34;
        int32_t sumi = dot32((const int8_t*)(wb + 2), (const int8_t*)(ab + 2));
        float delta = x86_mul(bpdq_o_f16_magic(rd16(wb)), bpdq_o_f16_magic(rd16(ab)));
        sumf = x86_add(sumf, x86_mul((float)sumi, delta));
    }
    return sumf;
}

/* AVX1 llamafile tile order T, one output cell: bench/bpd_gemm_q8_0_cpu.c:32-86.
 * Lane L accumulates the 4-element partial of elements 4L..4L+3 of every block:
 * scale = Ad*Bd, prod = scale*float(p_L), acc_L = prod + acc_L, then the hsum
 * ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)).  The values do not depend on the tile that
 * computes the cell; the bits of a NaN do, because the reference build's code for
 * each of the nine tile kernels puts different operands first.  Measured on that
 * build (one probe per operand pair, NaNs of both signs):
 *   Ad*Bd: Bd first in every tile;
 *   prod + acc: the accumulator first in the 1x1 tile, the product first in the others;
 *   the hsum: per cell, a mask of swapped additions, bit 0-3 for the pairs (a0,a4),
 *   (a2,a6), (a1,a5), (a3,a7) (set: the right one first), bit 4 for the left pair
 *   sum of the second level, bit 5 the right one, bit 6 the top addition.
 * t_tile_spec gives the cell's tile (bench/bpd_gemm_q8_0_cpu.c:159-207: 4, then 2,
 * then 1 rows / tokens) and its orders. */
typedef struct { int acc_first; unsigned mask; } t_spec;

static t_spec t_tile_spec(int r, int t, int m_weight, int m_tokens) {
    /* tile size along one axis and the index inside it */
    int full_r = m_weight / 4 * 4, full_t = m_tokens / 4 * 4;
    int RM = r < full_r ? 4 : (m_weight - full_r >= 2 && r < full_r + 2) ? 2 : 1;
    int RN = t < full_t ? 4 : (m_tokens - full_t >= 2 && t < full_t + 2) ? 2 : 1;
    int i = RM == 4 ? r % 4 : RM == 2 ? r - full_r : 0;
    int j = RN == 4 ? t % 4 : RN == 2 ? t - full_t : 0;
    t_spec s = {RM == 1 && RN == 1, 0u};
    if (RM == 4) s.mask = 0x12u;
    else if (RM == 2) s.mask = (RN == 1 || i == 0) ? 0u : 0x12u;
    else s.mask = RN == 4 ? 0x10u : RN == 2 ? (j == 0 ? 0x01u : 0x10u) : 0u;
    return s;
}

static inline float x86_add_sw(float a, float b, unsigned sw) { return sw ? x86_add(b, a) : x86_add(a, b); }

static float cell_q8_0_T(const uint8_t* w, const uint8_t* a, int n_blocks, t_spec sp) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int l = 0; l < n_blocks; l++) {
        const uint8_t* ab = a + (size_t)l * 34;
        const uint8_t* wb = w + (size_t)l * 34;
        float Bd = bpdq_o_f16_ldexp(rd16(ab));
        float Ad = bpdq_o_f16_ldexp(rd16(wb));
        float scale = x86_mul(Bd, Ad);
        for (int L = 0; L < 8; L++) {
            int32_t p = sse_quad((const int8_t*)(wb + 2) + 4 * L, (const int8_t*)(ab + 2) + 4 * L);
            float prod = x86_mul(scale, (float)p);
            acc[L] = sp.acc_first ? x86_add(acc[L], prod) : x86_add(prod, acc[L]);
        }
    }
    unsigned m = sp.mask;
    float l0 = x86_add_sw(acc[0], acc[4], m & 1u), l1 = x86_add_sw(acc[2], acc[6], m & 2u);
    float l2 = x86_add_sw(acc[1], acc[5], m & 4u), l3 = x86_add_sw(acc[3], acc[7], m & 8u);
    return x86_add_sw(x86_add_sw(l0, l1, m & 16u), x86_add_sw(l2, l3, m & 32u), m & 64u);
}

/* The cell as the 4-row tiles compute it (the tile of every cell of a 4x4 block). */
float bpdq_o_cell_q8_0_T(const uint8_t* w, const uint8_t* a, int n_blocks) {
    return cell_q8_0_T(w, a, n_blocks, t_tile_spec(0, 0, 4, 4));
}

/* bench/bpd_gemm_q8_0_cpu.c:159-207: every cell of out[token * m_weight + row]
 * is one tile cell; the tile shape never changes a cell's bits. */
void bpdq_o_dispatch_q8_0(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K, int order) {
    int k = K / 32;
    size_t bpr = (size_t)k * 34;
    for (int t = 0; t < m_tokens; t++)
        for (int r = 0; r < m_weight; r++) {
            const uint8_t* wr = Wq + (size_t)r * bpr;
            const uint8_t* xr = Xq + (size_t)t * bpr;
            out[(size_t)t * m_weight + r] = order == 'T' ? cell_q8_0_T(wr, xr, k, t_tile_spec(r, t, m_weight, m_tokens))
                                                         : bpdq_o_cell_q8_0_S(wr, xr, k);
        }
}

/* bench/bpd_cpu.c:4295-4315: out[m * N + n] = qdot(W row n, quant(X row m)). */
void bpdq_o_qmatmul_q8_0(const uint8_t* W, const float* X, float* out, int M, int N, int K, int order) {
    int nb = K / 32;
    size_t bpr = (size_t)nb * 34;
    uint8_t* Xq = (uint8_t*)malloc((size_t)M * bpr + 1);
    if (!Xq) return;
    for (int m = 0; m < M; m++) bpdq_o_quant_q8_0(X + (size_t)m * K, Xq + (size_t)m * bpr, K);
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++)
            out[(size_t)m * N + n] = order == 'P' ? bpdq_o_qdot_q8_0_P(W + (size_t)n * bpr, Xq + (size_t)m * bpr, nb)
                                                  : bpdq_o_qdot_q8_0_S(W + (size_t)n * bpr, Xq + (size_t)m * bpr, nb);
    free(Xq);
}

/* bench/bpd_cpu.c:4429-4452 (AVX1: quantize X, then the dispatcher, order T) and
 * :4455-4458 (scalar build: bpd_qmatmul_q8_0_cpu(W, X, out, mt, mw, K), order S). */
void bpdq_o_qmatmul_q8_0_llamafile(const uint8_t* W, const float* X, float* out, int m_weight, int m_tokens, int K, int order) {
    if (order != 'T') {
        bpdq_o_qmatmul_q8_0(W, X, out, m_tokens, m_weight, K, 'S');
        return;
    }
    int k = K / 32;
    size_t bpr = (size_t)k * 34;
    uint8_t* Xq = (uint8_t*)malloc((size_t)m_tokens * bpr + 1);
    if (!Xq) return;
    for (int i = 0; i < m_tokens; i++) bpdq_o_quant_q8_0(X + (size_t)i * K, Xq + (size_t)i * bpr, K);
    bpdq_o_dispatch_q8_0(W, Xq, out, m_weight, m_tokens, K, 'T');
    free(Xq);
}

/* -------------------------------------------------- padded Q8 layout --- */

/* q8_pad64_coalesced, inference/llamatov_c_inference.py:88-100, in float32 as
 * numpy evaluates it (NEP 50: float32 array op Python float stays float32):
 * amax = max(max|x|, 1e-10f); d = amax / 127; q = clip(rint(x / d), -128, 127)
 * (np.round is round-half-even, as rintf in the default mode); d stored as RNE
 * binary16; record (b, n) at byte (b*N + n)*64 = {d16, 0, 0, q[32], 0 x 28}. */
void bpdq_o_q8_pad64(const float* x, uint8_t* out, int N, int K) {
    int nb = K / 32;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < nb; b++) {
            const float* xb = x + (size_t)n * K + (size_t)b * 32;
            uint8_t* o = out + ((size_t)b * N + n) * 64;
            float amax = 0.0f;
            int has_nan = 0;
            for (int j = 0; j < 32; j++) {
                float a = fabsf(xb[j]);
                if (isnan(a)) has_nan = 1;
                else if (a > amax) amax = a;
            }
            memset(o, 0, 64);
            if (has_nan) {
                /* numpy's max, clip and /127 carry the NaN into d, so every x/d is
                 * NaN and casts to 0; d's float16 is 0x7E00 for the default NaN (a
                 * payload survives numpy's SIMD max at some positions only) */
                const uint16_t h = 0x7E00;
                memcpy(o, &h, 2);
                continue;
            }
            if (amax < 1e-10f) amax = 1e-10f;
            float d = amax / 127.0f;
            uint16_t h = bpdq_o_f32_to_f16(d);
            memcpy(o, &h, 2);
            for (int j = 0; j < 32; j++) {
                float q = rintf(xb[j] / d);
                if (isnan(q)) q = 0.0f;  /* Inf/Inf (amax = Inf): clip keeps the NaN, the int8 cast gives 0 */
                if (q < -128.0f) q = -128.0f;
                if (q > 127.0f) q = 127.0f;
                o[4 + j] = (uint8_t)x86_f32_to_i8(q);
            }
        }
}

/* ------------------------------------------------- multi-threaded wrappers */

typedef struct {
    int kind, order, K, mw, mt;
    const uint8_t* a;
    const uint8_t* b;
    float* out;
    int r0, r1;
} mt_job;

static void* mt_run(void* p) {
    mt_job* j = (mt_job*)p;
    if (j->kind == 0) {
        bpdq_o_dequant_q4k(j->a + (size_t)j->r0 * 144, j->out + (size_t)j->r0 * 256, j->r1 - j->r0);
    } else if (j->kind == 1) {
        int nb = j->K / 256;
        for (int r = j->r0; r < j->r1; r++) j->out[r] = q4k_q8k_row(j->a + (size_t)r * nb * 144, j->b, nb, j->order);
    } else if (j->kind == 3) {
        int nb = j->K / 256;
        for (int r = j->r0; r < j->r1; r++) j->out[r] = q6k_q8k_row(j->a + (size_t)r * nb * 210, j->b, nb, j->order);
    } else {
        int k = j->K / 32;
        size_t bpr = (size_t)k * 34;
        for (int t = 0; t < j->mt; t++)
            for (int r = j->r0; r < j->r1; r++)
                j->out[(size_t)t * j->mw + r] =
                    j->order == 'T' ? cell_q8_0_T(j->a + (size_t)r * bpr, j->b + (size_t)t * bpr, k,
                                                  t_tile_spec(r, t, j->mw, j->mt))
                                    : bpdq_o_cell_q8_0_S(j->a + (size_t)r * bpr, j->b + (size_t)t * bpr, k);
    }
    return NULL;
}

static void mt_launch(mt_job proto, int n, int nthreads) {
    enum { MAXT = 256 };
    if (nthreads < 1) nthreads = 1;
    if (nthreads > MAXT) nthreads = MAXT;
    if (nthreads > n) nthreads = n > 0 ? n : 1;
    mt_job jobs[MAXT];
    pthread_t th[MAXT];
    int ok[MAXT];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = proto;
        jobs[t].r0 = (int)((long long)n * t / nthreads);
        jobs[t].r1 = (int)((long long)n * (t + 1) / nthreads);
        ok[t] = t > 0 && pthread_create(&th[t], NULL, mt_run, &jobs[t]) == 0;
        if (t > 0 && !ok[t]) mt_run(&jobs[t]);
    }
    mt_run(&jobs[0]);
    for (int t = 1; t < nthreads; t++)
        if (ok[t]) pthread_join(th[t], NULL);
}

void bpdq_o_dequant_q4k_mt(const uint8_t* q, float* out, int n_blocks, int nthreads) {
    mt_job p = {0};
    p.kind = 0; p.a = q; p.out = out;
    mt_launch(p, n_blocks, nthreads);
}

void bpdq_o_qmatmul_q4k_q8k_mt(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, int nthreads) {
    mt_job p = {0};
    p.kind = 1; p.a = w; p.b = xq; p.out = y; p.K = K; p.order = order;
    mt_launch(p, M, nthreads);
}

void bpdq_o_dispatch_q8_0_mt(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K, int order, int nthreads) {
    mt_job p = {0};
    p.kind = 2; p.a = Wq; p.b = Xq; p.out = out; p.K = K; p.order = order; p.mw = m_weight; p.mt = m_tokens;
    mt_launch(p, m_weight, nthreads);
}

void bpdq_o_qmatmul_q6k_q8k_mt(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, int nthreads) {
    mt_job p = {0};
    p.kind = 3; p.a = w; p.b = xq; p.out = y; p.K = K; p.order = order;
    mt_launch(p, M, nthreads);
}

/* ==========================================================================
 * The decode step.
 * ========================================================================== */

/* expf by the method the C library uses on x86-64 glibc with FMA (Szabolcs
 * Nagy's table-driven expf, ARM optimized-routines math/expf.c): see
 * bpd_substrate_amd/csrc/bpdq_math.h, whose device code runs the same steps. */
static const uint64_t expf_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

void bpdq_o_expf_table(uint64_t* out) { memcpy(out, expf_tab, sizeof expf_tab); }

float bpdq_o_expf_nagy(float x) {
    const double N = 32.0, InvLn2N = 0x1.71547652b82fep+0 * N, Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / (N * N * N), C1 = 0x1.ebfce50fac4f3p-3 / (N * N),
                 C2 = 0x1.62e42ff0c52d6p-1 / N;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = fma(InvLn2N, xd, Shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= Shift;
    const double r = fma(InvLn2N, xd, -kd);
    const uint64_t t = expf_tab[ki & 31] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

typedef struct {
    uint32_t start, step;
    uint64_t bad;
    uint32_t first_bad;
} expf_job;

static float (*volatile libm_expf)(float) = expf;

static void* expf_run(void* p) {
    expf_job* j = (expf_job*)p;
    for (uint64_t u = j->start; u <= 0xFFFFFFFFull; u += j->step) {
        float x;
        const uint32_t v = (uint32_t)u;
        memcpy(&x, &v, 4);
        if (x != x) continue;
        const float a = libm_expf(x), b = bpdq_o_expf_nagy(x);
        if (memcmp(&a, &b, 4) != 0) {
            if (j->bad == 0) j->first_bad = v;
            j->bad++;
        }
    }
    return NULL;
}

uint64_t bpdq_o_expf_mismatches(int nthreads, uint32_t stride, uint32_t* first_bad) {
    enum { MAXJ = 64 };
    if (nthreads < 1) nthreads = 1;
    if (nthreads > MAXJ) nthreads = MAXJ;
    if (stride < 1) stride = 1;
    expf_job jobs[MAXJ];
    pthread_t th[MAXJ];
    int ok[MAXJ];
    for (int t = 0; t < nthreads; t++) {
        jobs[t].start = (uint32_t)t * stride;
        jobs[t].step = (uint32_t)nthreads * stride;
        jobs[t].bad = 0;
        jobs[t].first_bad = 0;
        ok[t] = t > 0 && pthread_create(&th[t], NULL, expf_run, &jobs[t]) == 0;
    }
    for (int t = 1; t < nthreads; t++)
        if (!ok[t]) expf_run(&jobs[t]);
    expf_run(&jobs[0]);
    uint64_t bad = 0;
    *first_bad = 0;
    for (int t = 0; t < nthreads; t++) {
        if (ok[t]) pthread_join(th[t], NULL);
        if (jobs[t].bad && !bad) *first_bad = jobs[t].first_bad;
        bad += jobs[t].bad;
    }
    return bad;
}

void bpdq_o_libm_expf(const float* x, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = libm_expf(x[i]);
}

/* bench/bpd_cpu.c:4959-4986 */
void bpdq_o_rmsnorm(const float* x, const float* w, float* y, int n, float eps) {
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
    const float mean = (float)(sum / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

/* bench/bpd_cpu.c:5146-5184 (NORM pairs), no frequency factors, n_dims = head_dim. */
void bpdq_o_rope_norm(float* t, int n_heads, int head_dim, int pos, float base) {
    const float theta_scale = powf(base, -2.0f / (float)head_dim);
    for (int hh = 0; hh < n_heads; hh++) {
        float* p = t + (size_t)hh * head_dim;
        float theta = (float)pos;
        for (int i0 = 0; i0 < head_dim; i0 += 2) {
            const float c = cosf(theta), s = sinf(theta);
            const float x0 = p[i0], x1 = p[i0 + 1];
            p[i0] = x0 * c - x1 * s;
            p[i0 + 1] = x0 * s + x1 * c;
            theta *= theta_scale;
        }
    }
}

/* bench/bpd_cpu.c:5370-5440 for one query token at position pos, over all
 * max_seq cache rows with the causal mask (rows > pos weigh exp(-1e38 - max)). */
void bpdq_o_gqa_attn(const float* q, const float* kc, const float* vc, float* out, int max_seq, int pos, int H,
                     int HKV, int D, float scale) {
    const int grp = H / HKV, row = HKV * D;
    float* sc = (float*)malloc(sizeof(float) * (size_t)max_seq);
    for (int h = 0; h < H; h++) {
        const int kvh = h / grp;
        const float* pq = q + (size_t)h * D;
        for (int j = 0; j < max_seq; j++) {
            const float* pk = kc + (size_t)j * row + (size_t)kvh * D;
            float s = 0.0f;
            for (int d = 0; d < D; d++) s += pq[d] * pk[d];
            sc[j] = s;
        }
        float mx = -1e38f;
        for (int j = 0; j < max_seq; j++) {
            const float sv = j <= pos ? sc[j] * scale : -1e38f;
            sc[j] = sv;
            if (sv > mx) mx = sv;
        }
        float sum = 0.0f;
        for (int j = 0; j < max_seq; j++) {
            const float e = expf(sc[j] - mx);
            sc[j] = e;
            sum += e;
        }
        const float inv = sum == 0.0f ? 0.0f : 1.0f / sum;
        for (int j = 0; j < max_seq; j++) sc[j] *= inv;
        float* o = out + (size_t)h * D;
        for (int d = 0; d < D; d++) o[d] = 0.0f;
        for (int j = 0; j < max_seq; j++) {
            const float* pv = vc + (size_t)j * row + (size_t)kvh * D;
            for (int d = 0; d < D; d++) o[d] += pv[d] * sc[j];
        }
    }
    free(sc);
}

/* bench/bpd_cpu.c:5504-5507 */
void bpdq_o_swiglu(const float* g, const float* u, float* y, int n) {
    for (int i = 0; i < n; i++) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* bench/bpd_cpu.c:4512-4526 */
int bpdq_o_argmax(const float* x, int n) {
    float best = x[0];
    int bi = 0;
    for (int k = 1; k < n; k++)
        if (x[k] > best) {
            best = x[k];
            bi = k;
        }
    return bi;
}

/* The fp32 head of the decode step (no reference source): lane l of a 64-wide
 * wave sums W[r][l + 64 i] * x[l + 64 i] over i, then xor-32..1 pair sums. */
void bpdq_o_gemv_f32_wave(const float* W, const float* x, float* y, int N, int K) {
    for (int r = 0; r < N; r++) {
        float p[64];
        for (int l = 0; l < 64; l++) {
            float a = 0.0f;
            for (int k = l; k < K; k += 64) a = a + W[(size_t)r * K + k] * x[k];
            p[l] = a;
        }
        for (int m = 32; m >= 1; m >>= 1) {
            float t[64];
            for (int l = 0; l < 64; l++) t[l] = p[l] + p[l ^ m];
            memcpy(p, t, sizeof p);
        }
        y[r] = p[0];
    }
}

/* y[N] = W[N][K] a[K] in the step's weight format. */
static void step_gemv(int fmt, const uint8_t* W, const float* a, float* y, int N, int K) {
    if (fmt == 0) {
        uint8_t* aq = (uint8_t*)malloc((size_t)(K / 32) * 34);
        bpdq_o_quant_q8_0(a, aq, K);
        bpdq_o_dispatch_q8_0(W, aq, y, N, 1, K, 'T');
        free(aq);
    } else {
        uint8_t* aq = (uint8_t*)malloc((size_t)(K / 256) * 292);
        bpdq_o_quant_q8_k(a, aq, K);
        if (fmt == 3 || fmt == 4)
            bpdq_o_qmatmul_q6k_q8k(W, aq, y, N, K, fmt == 4 ? 1 : 0);
        else
            bpdq_o_qmatmul_q4k_q8k(W, aq, y, N, K, fmt == 2 ? 1 : 0);
        free(aq);
    }
}

/* bench/bpd_cpu.c:5146-5184, one token */
void bpdq_o_rope_norm_freqs(float* t, int n_heads, int head_dim, int pos, float base, int n_dims,
                            const float* freqs) {
    const float theta_scale = powf(base, -2.0f / (float)n_dims);
    for (int hh = 0; hh < n_heads; hh++) {
        float* p = t + (size_t)hh * head_dim;
        float theta = (float)pos;
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const float ff = freqs ? freqs[i0 / 2] : 1.0f;
            const float te = theta / ff;
            const float c = cosf(te), s = sinf(te);
            const float x0 = p[i0], x1 = p[i0 + 1];
            p[i0] = x0 * c - x1 * s;
            p[i0 + 1] = x0 * s + x1 * c;
            theta *= theta_scale;
        }
    }
}

/* The composition of bpd_llama_block_cpu (bench/bpd_cpu.c:5611-5737) over the
 * layers and the head of bpd_llama_forward_cpu (:5779-5792) for one token. */
int bpdq_o_llama_step_ext(const bpdq_o_step_opts* o, const bpdq_o_layer* layers, const bpdq_o_cfg* cfg,
                          void* const* k_cache, void* const* v_cache, int pos, const float* emb,
                          const float* out_norm, const uint8_t* lm, const float* lm_f32, int lm_N, float* x,
                          float* h, float* logits) {
    const int E = cfg->n_embd, H = cfg->n_head, HKV = cfg->n_head_kv, D = cfg->head_dim, F = cfg->ff_dim;
    const int row = HKV * D, S = cfg->max_seq;
    float* q = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* k = (float*)malloc(sizeof(float) * (size_t)row);
    float* v = (float*)malloc(sizeof(float) * (size_t)row);
    float* att = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* t = (float*)malloc(sizeof(float) * (size_t)E);
    float* g = (float*)malloc(sizeof(float) * (size_t)F);
    float* u = (float*)malloc(sizeof(float) * (size_t)F);
    float* kf = o->kv_f16 ? (float*)malloc(sizeof(float) * (size_t)S * row) : NULL;
    float* vf = o->kv_f16 ? (float*)malloc(sizeof(float) * (size_t)S * row) : NULL;
    memcpy(x, emb, sizeof(float) * (size_t)E);
    const float scale = 1.0f / sqrtf((float)D);
    for (int l = 0; l < cfg->n_layers; l++) {
        const bpdq_o_layer* w = &layers[l];
        const int* f = o->fmts + 7 * l;
        bpdq_o_rmsnorm(x, w->attn_norm, h, E, cfg->eps);
        step_gemv(f[0], w->q, h, q, H * D, E);
        step_gemv(f[1], w->k, h, k, row, E);
        step_gemv(f[2], w->v, h, v, row, E);
        if (w->q_bias) for (int i = 0; i < H * D; i++) q[i] = q[i] + w->q_bias[i];
        if (w->k_bias) for (int i = 0; i < row; i++) k[i] = k[i] + w->k_bias[i];
        if (w->v_bias) for (int i = 0; i < row; i++) v[i] = v[i] + w->v_bias[i];
        bpdq_o_rope_norm_freqs(q, H, D, pos, cfg->rope_theta, o->rope_dim, o->rope_freqs);
        bpdq_o_rope_norm_freqs(k, HKV, D, pos, cfg->rope_theta, o->rope_dim, o->rope_freqs);
        if (o->kv_f16) {
            uint16_t* kc = (uint16_t*)k_cache[l];
            uint16_t* vc = (uint16_t*)v_cache[l];
            for (int i = 0; i < row; i++) {
                kc[(size_t)pos * row + i] = bpdq_o_f32_to_f16(k[i]);
                vc[(size_t)pos * row + i] = bpdq_o_f32_to_f16(v[i]);
            }
            for (size_t i = 0; i < (size_t)S * row; i++) {
                kf[i] = bpdq_o_f16_magic(kc[i]);
                vf[i] = bpdq_o_f16_magic(vc[i]);
            }
            bpdq_o_gqa_attn(q, kf, vf, att, S, pos, H, HKV, D, scale);
        } else {
            float* kc = (float*)k_cache[l];
            float* vc = (float*)v_cache[l];
            memcpy(kc + (size_t)pos * row, k, sizeof(float) * (size_t)row);
            memcpy(vc + (size_t)pos * row, v, sizeof(float) * (size_t)row);
            bpdq_o_gqa_attn(q, kc, vc, att, S, pos, H, HKV, D, scale);
        }
        step_gemv(f[3], w->o, att, t, E, H * D);
        for (int i = 0; i < E; i++) x[i] = x[i] + t[i];
        bpdq_o_rmsnorm(x, w->ffn_norm, h, E, cfg->eps);
        step_gemv(f[4], w->gate, h, g, F, E);
        step_gemv(f[5], w->up, h, u, F, E);
        bpdq_o_swiglu(g, u, g, F);
        step_gemv(f[6], w->down, g, t, E, F);
        for (int i = 0; i < E; i++) x[i] = x[i] + t[i];
    }
    bpdq_o_rmsnorm(x, out_norm, h, E, cfg->eps);
    if (lm)
        step_gemv(o->lm_fmt, lm, h, logits, lm_N, E);
    else
        bpdq_o_gemv_f32_wave(lm_f32, h, logits, lm_N, E);
    free(q); free(k); free(v); free(att); free(t); free(g); free(u); free(kf); free(vf);
    return bpdq_o_argmax(logits, lm_N);
}

int bpdq_o_llama_step(int fmt, const bpdq_o_layer* layers, const bpdq_o_cfg* cfg, float* const* k_cache,
                      float* const* v_cache, int pos, const float* emb, const float* out_norm, const uint8_t* lm,
                      const float* lm_f32, int lm_N, float* x, float* h, float* logits) {
    const int L = cfg->n_layers > 0 ? cfg->n_layers : 1;
    int* fmts = (int*)malloc(sizeof(int) * 7 * (size_t)L);
    for (int i = 0; i < 7 * L; i++) fmts[i] = fmt;
    const bpdq_o_step_opts o = {fmts, fmt, cfg->head_dim, NULL, 0};
    const int tok = bpdq_o_llama_step_ext(&o, layers, cfg, (void* const*)k_cache, (void* const*)v_cache, pos, emb,
                                          out_norm, lm, lm_f32, lm_N, x, h, logits);
    free(fmts);
    return tok;
}
