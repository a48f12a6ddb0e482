// llama.hip — the decode step of a llama-family model on gfx950
// (include/bpdq_llama.h): kernels, the per-step launch sequence, and the
// generate_token ABI of inference/llamatov_c_inference.py:15-83.
//
//   k_residual_rmsnorm  x = x_in (+ add); h = rmsnorm(x) * w; Q8_0(h)   one workgroup
//   k_attn_small        attention for pos < 64: one workgroup per query head does q/k/v
//                       bias, RoPE (NORM pairs), the K/V cache row write, scores,
//                       softmax, P.V and Q8_0(out)
//   k_attn_scores       longer contexts: bias, RoPE, cache row write and the scores,
//                       per (kv head, 64 rows), the k rows read once into LDS
//   k_attn_pv           longer contexts: softmax and P.V per (head, 16 or 32 columns),
//                       one wave running the chains while four stream V
//   k_swiglu            silu(gate) * up, Q8_0 (padded Q8 weights; with Q4_K the
//                       gate/up GEMV applies it to its own outputs)
//   k_argmax            first index of the maximum logit
//   k_gemv_f32          fp32 head (tied embeddings)
// The seven GEMVs of a layer are the padded-Q8 tile-order product (q8_0.hip) or
// the fused Q4_K x Q8_K product (q4k.hip).
//
// Every fp32 operation follows the reference's CPU block in order
// (bench/bpd_cpu.c:5611-5737 and the helpers it calls), so with Q8 weights the
// step is bit-identical to it:
//   - sums that the reference runs sequentially (an attention score over
//     head_dim, the softmax denominator, each output of P.V) run sequentially
//     here, in one lane, in the same order;
//   - max, amax and argmax are exact in any order;
//   - expf is the libm method restated in bpdq_math.h; cos/sin of the rotary
//     angles come from the host's libm (sincosf, which is what the reference's
//     compiled cosf/sinf pair calls) through a kernel argument;
//   - the RMSNorm sum of squares is binary64 like the reference's; its
//     parallel sum is used only when an error bound proves it gives the same
//     fp32 mean as the reference's sequential binary64 sum.
#include <algorithm>
#include <climits>
#include <initializer_list>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/bpdq.h"
#include "../../include/bpdq_llama.h"
#include "bpdq_device.h"
#include "bpdq_launch.h"
#include "bpdq_math.h"

namespace bpdq {

constexpr int kMaxEmbd = 16384;  // the residual row stays in LDS (64 KB)
constexpr int kNormThreads = 1024;
constexpr int kNormChunks = kMaxEmbd / (4 * kNormThreads);  // float4 chunks per thread
constexpr int kMaxHeadDim = 256;
constexpr int kMaxCtx = 32768;  // one head's scores stay in LDS (128 KB)

// ----------------------------------------------------------------------------
// Residual add + RMSNorm + Q8_0, one workgroup for the whole row
// (bpd_add_f32_cpu, bench/bpd_cpu.c:5466; bpd_rmsnorm_llama_cpu, :4959-4986):
//   x = x_in + add;  mean = (float)(sum_i (double)x_i^2 / n)   (sequential in the reference)
//   scale = 1 / sqrtf(mean + eps);  h_i = (x_i * scale) * w_i.
// The squares are exact in binary64.  Any summation order of n non-negative
// terms is within (n-1) 2^-53 S of the exact sum S, so the reference's
// sequential sum lies within E = 4 n 2^-53 S_tree of this kernel's tree sum.
// If (float)((S_tree - E)/n) == (float)((S_tree + E)/n), rounding monotonicity
// pins the reference's mean to that value; otherwise lane 0 redoes the
// reference's sequential sum from the row kept in LDS.
// ----------------------------------------------------------------------------
// Thread t holds float4 chunks t, t + NT, ... of the row (MAXC at most), with
// the norm weight loaded alongside.  Q8_0 blocks are 8 consecutive lanes.
// xk (or NULL) receives Q8_K blocks of h, the bytes k_quant_q8k writes: chunk
// c of a thread is lane c % 64 of block c / 64, so each block is one whole wave
// (n % 256 == 0 when xk is given).  Workgroup b normalizes row b of row-major
// [rows][n] tensors (bpd_rmsnorm_llama_cpu's n_rows).
template <int NT, int MAXC>
__global__ __launch_bounds__(NT) void k_residual_rmsnorm(const float* x_in, const float* __restrict__ add,
                                                         float* x_out, const float* __restrict__ w,
                                                         float* __restrict__ h, uint8_t* __restrict__ xq,
                                                         uint8_t* __restrict__ xk, int n, float eps) {
    extern __shared__ float4 xs4[];
    __shared__ double wsum[NT / 64];
    __shared__ float sh_scale;
    const int tid = threadIdx.x, nc = n >> 2;
    {
        const int64_t row = blockIdx.x, ro = row * n;
        x_in += ro;
        if (add != nullptr) add += ro;
        if (x_out != nullptr) x_out += ro;
        if (h != nullptr) h += ro;
        if (xq != nullptr) xq += row * (n / 32) * kQ80Bytes;
        if (xk != nullptr) xk += row * (n / 256) * kQ8KBytes;
    }
    const float4* x4 = reinterpret_cast<const float4*>(x_in);
    const float4* a4 = reinterpret_cast<const float4*>(add);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[MAXC], wv[MAXC];
#pragma unroll
    for (int j = 0; j < MAXC; j++) {
        const int c = tid + j * NT;
        if (c < nc) {
            v[j] = x4[c];
            wv[j] = w4[c];
            if (add != nullptr) {
                const float4 a = a4[c];
                v[j] = make_float4(v[j].x + a.x, v[j].y + a.y, v[j].z + a.z, v[j].w + a.w);
            }
        }
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < MAXC; j++) {
        const int c = tid + j * NT;
        if (c < nc) {
            xs4[c] = v[j];
            if (x_out != nullptr) reinterpret_cast<float4*>(x_out)[c] = v[j];
            s += (double)v[j].x * v[j].x + (double)v[j].y * v[j].y + (double)v[j].z * v[j].z +
                 (double)v[j].w * v[j].w;
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    if ((tid & 63) == 0) wsum[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        double S = 0.0;
        for (int i = 0; i < NT / 64; i++) S += wsum[i];
        sh_scale = rms_scale(S, reinterpret_cast<const float*>(xs4), n, eps);
    }
    __syncthreads();
    const float scale = sh_scale;
#pragma unroll
    for (int j = 0; j < MAXC; j++) {
        const int c = tid + j * NT;
        if (c < nc) {
            const float4 x = v[j], ww = wv[j];
            const float4 y = make_float4((x.x * scale) * ww.x, (x.y * scale) * ww.y, (x.z * scale) * ww.z,
                                         (x.w * scale) * ww.w);
            if (h != nullptr) reinterpret_cast<float4*>(h)[c] = y;
            // n % 32 == 0 and NT % 8 == 0: the 8 chunks of a block are 8 aligned lanes
            if (xq != nullptr) q8_0_quad_store(y, xq + (int64_t)(c >> 3) * kQ80Bytes, c & 7);
            if (xk != nullptr) q8k_wave_store(y, xk + (int64_t)(c >> 6) * kQ8KBytes, c & 63);
        }
    }
}

// The FFN norm of a step whose O GEMV added its rows into the residual row x
// and left binary64 partial sums of squares (launch_q4k_res): wave b quantizes
// block b of h = (x * scale) * w to Q8_K for the gate/up GEMV, the scale from
// the partials (rms_scale), so xk holds k_residual_rmsnorm's bytes.
constexpr int kNormParts = 16;  // partials per lane held in registers (producers write <= 1024)
__global__ __launch_bounds__(64) void k_norm_q8k(NormIn nin, uint8_t* __restrict__ xk) {
    const int lane = threadIdx.x, c = blockIdx.x * 64 + lane;
    // every load issued before any is used: x and w, then the partials
    // unconditionally (past npart: a re-read of the last one, then 0)
    const float4 x = reinterpret_cast<const float4*>(nin.x)[c];
    const float4 w = reinterpret_cast<const float4*>(nin.w)[c];
    double pp[kNormParts];
#pragma unroll
    for (int k = 0; k < kNormParts; k++) {
        const double v = nin.part[min(lane + 64 * k, max(nin.npart - 1, 0))];
        pp[k] = lane + 64 * k < nin.npart ? v : 0.0;
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < kNormParts; k++) s += pp[k];
    for (int i = lane + 64 * kNormParts; i < nin.npart; i += 64) s += nin.part[i];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);  // the same S in every lane
    const float scale = rms_scale(s, nin.x, gridDim.x * 256, nin.eps);
    const float4 y = make_float4((x.x * scale) * w.x, (x.y * scale) * w.y, (x.z * scale) * w.z, (x.w * scale) * w.w);
    q8k_wave_store(y, xk + (int64_t)blockIdx.x * kQ8KBytes, lane);
}

// ----------------------------------------------------------------------------
// Decode attention of query head blockIdx.x at position pos, with the bias,
// RoPE and K/V cache write of the new row folded in:
//   bias: q, k, v = projection + bias (when given), before RoPE;
//   RoPE (bpd_rope_norm_freqs_cpu, bench/bpd_cpu.c:5146-5184, no frequency
//     factors): pair j of a head rotates elements 2j, 2j+1 by pos*theta_scale^j,
//     y0 = x0*c - x1*s, y1 = x0*s + x1*c (each product rounded, then the sum),
//     cos/sin from the host;
//   the new k and v rows go to cache row pos (bpd_kv_cache_write_cpu, :5204),
//     written by the first query head of each group; every head of the group
//     takes row pos from its own LDS copy, so no head reads a row another
//     workgroup is writing;
//   attention (bpd_gqa_attn_cpu, :5370-5440, post-scaled batch softmax) over
//     rows 0..pos:
//   s_j = sum_d q_d k_jd (sequential over d);  v_j = s_j * scale
//   m = max(-1e38, v_j);  e_j = expf(v_j - m);  S = sum_j e_j (sequential over j)
//   w_j = e_j * (S == 0 ? 0 : 1/S);  out_d = sum_j v_jd w_j (sequential over j)
// The reference also visits rows pos+1..max_seq-1 with weight exp(-1e38 - m) =
// 0; for finite cache contents those add exact zeros, so stopping at pos gives
// the same bits.  Scores live in LDS.
// ----------------------------------------------------------------------------
struct RopeTab {
    float c[kMaxHeadDim / 2];
    float s[kMaxHeadDim / 2];
};

// K/V cache elements: fp32, or binary16 with the reference's conversions
// (bpd_kv_cache_write_f16_cpu, bench/bpd_cpu.c:5240, stores f32_to_f16, :4049,
// RNE with NaN payloads truncated and made nonzero; the block reads the cache
// back through f16_to_f32, :3928, whose magic-number form keeps a NaN's
// payload and sets the quiet bit).
template <typename CT>
struct Cache;
// ldr loads 4 consecutive elements raw and cvt turns them into fp32, so a
// prefetch can hold raw loads in flight and convert them only when used.
template <>
struct Cache<float> {
    using Raw = float4;
    static __device__ __forceinline__ Raw ldr(const float* p) { return *reinterpret_cast<const float4*>(p); }
    static __device__ __forceinline__ float4 cvt(Raw r) { return r; }
    static __device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
    static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
    static __device__ __forceinline__ float rt(float v) { return v; }  // the value as read back
};
__device__ __forceinline__ uint32_t f32_to_f16_ref(float v) {
    const uint32_t u = __float_as_uint(v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7C00u | ((u & 0x7FFFFFu) >> 13) | 1u;
    return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: RNE, subnormals, overflow to Inf
}
__device__ __forceinline__ float f16_to_f32_ref(uint32_t h) {
    return f16_is_nan(h) ? f16_nan_x86(h) : f16_ieee(h);
}
template <>
struct Cache<uint16_t> {
    using Raw = uint2;
    static __device__ __forceinline__ Raw ldr(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
    static __device__ __forceinline__ float4 cvt(Raw u) {
        return make_float4(f16_to_f32_ref(u.x & 0xFFFFu), f16_to_f32_ref(u.x >> 16), f16_to_f32_ref(u.y & 0xFFFFu),
                           f16_to_f32_ref(u.y >> 16));
    }
    static __device__ __forceinline__ float4 ld4(const uint16_t* p) { return cvt(ldr(p)); }
    static __device__ __forceinline__ void st(uint16_t* p, float v) { *p = (uint16_t)f32_to_f16_ref(v); }
    static __device__ __forceinline__ float rt(float v) { return f16_to_f32_ref(f32_to_f16_ref(v)); }
};

struct AttnIn {
    const float *q, *knew, *vnew;  // projections of this token (before bias and RoPE)
    const float *bq, *bk, *bv;     // biases or NULL
    void *kc, *vc;                 // this layer's caches, [max_seq][row] of the cache type
    int group, row, D, pos;
    float scale;
    int rot;                       // pairs 0..rot-1 of a head rotate, the rest pass through
};

// Bias + RoPE of query head `head` into qs (unless NULL) and, with `with_kv`,
// of the new k row into ks and the new v row into vs (all LDS), as the cache
// will give them back.  With `write`, the thread that computes an element of
// the new k or v row also stores it to cache row pos.
template <typename CT>
__device__ __forceinline__ void rope_rows(const AttnIn& a, const RopeTab& tab, int head, int kvh, float* qs,
                                          float* ks, float* vs, bool with_kv, bool write) {
    const int64_t qo = (int64_t)head * a.D, ko = (int64_t)kvh * a.D;
    CT* kc = static_cast<CT*>(a.kc) + (int64_t)a.pos * a.row + ko;
    CT* vc = static_cast<CT*>(a.vc) + (int64_t)a.pos * a.row + ko;
    for (int p = threadIdx.x; p < a.D / 2; p += blockDim.x) {
        const int i = 2 * p;
        const bool rot = p < a.rot;
        const float c = tab.c[p], sn = tab.s[p];
        if (qs != nullptr) {
            float x0 = a.q[qo + i], x1 = a.q[qo + i + 1];
            if (a.bq != nullptr) {
                x0 = x0 + a.bq[qo + i];
                x1 = x1 + a.bq[qo + i + 1];
            }
            qs[i] = rot ? x0 * c - x1 * sn : x0;
            qs[i + 1] = rot ? x0 * sn + x1 * c : x1;
        }
        if (with_kv) {
            float k0 = a.knew[ko + i], k1 = a.knew[ko + i + 1];
            if (a.bk != nullptr) {
                k0 = k0 + a.bk[ko + i];
                k1 = k1 + a.bk[ko + i + 1];
            }
            const float y0 = rot ? k0 * c - k1 * sn : k0, y1 = rot ? k0 * sn + k1 * c : k1;
            ks[i] = Cache<CT>::rt(y0);
            ks[i + 1] = Cache<CT>::rt(y1);
            if (write) {
                Cache<CT>::st(kc + i, y0);
                Cache<CT>::st(kc + i + 1, y1);
            }
        }
    }
    if (with_kv)
        for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
            float vv = a.vnew[ko + d];
            if (a.bv != nullptr) vv = vv + a.bv[ko + d];
            vs[d] = Cache<CT>::rt(vv);
            if (write) Cache<CT>::st(vc + d, vv);
        }
}

// Sequential dot products of q with one k row: s = s + q_d * k_d, d ascending.
__device__ __forceinline__ float dot_step(float s, float4 q, float4 k) {
    s = s + q.x * k.x;
    s = s + q.y * k.y;
    s = s + q.z * k.z;
    return s + q.w * k.w;
}
template <int D4>
__device__ __forceinline__ float dot_regs(const float4* qs4, const float4 (&k)[D4]) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < D4; i++) s = dot_step(s, qs4[i], k[i]);
    return s;
}
__device__ __forceinline__ float dot_ptr(const float4* qs4, const float4* k, int D4) {
    float s = 0.0f;
#pragma unroll 8
    for (int i = 0; i < D4; i++) s = dot_step(s, qs4[i], k[i]);
    return s;
}

// Block-wide max of the scaled scores, as the reference's scan keeps it
// (start at -1e38, take v when v > max): exact in any order.  No value is NaN
// (a scan that starts below every score never takes one).  Inside a wave the
// reduction runs on DPP moves (quad_perm, row_half_mirror, row_mirror: the
// max of each 16-lane row) and four readlanes.
__device__ __forceinline__ float max_gt(float a, float b) { return b > a ? b : a; }
template <int NT>
__device__ __forceinline__ float block_max(float m, float* red) {
    m = max_gt(m, dpp_f<0xB1>(m));   // quad_perm [1,0,3,2]
    m = max_gt(m, dpp_f<0x4E>(m));   // quad_perm [2,3,0,1]
    m = max_gt(m, dpp_f<0x141>(m));  // row_half_mirror
    m = max_gt(m, dpp_f<0x140>(m));  // row_mirror
    m = max_gt(max_gt(readlane_f(m, 0), readlane_f(m, 16)), max_gt(readlane_f(m, 32), readlane_f(m, 48)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) mx = max_gt(mx, red[w]);
    return mx;
}

// Sequential fp32 sums read from LDS in groups of G float4, the next group's
// reads issued before the current group's adds (sched_barrier keeps the
// compiler from sinking them below the adds).  A wave's VALU issue is the
// limit here: a dependent add from registers takes ~4.4 cycles and each LDS
// read instruction ~10, so 16-float4 groups (one read per 4 adds, few waits)
// run at ~8.3 cycles per element against ~10 for 8-float4 groups (measured,
// one wave, 2,048 elements).
template <int G>
__device__ __forceinline__ void sum_group(float& sum, const float4 (&v)[G]) {
#pragma unroll
    for (int i = 0; i < G; i++) {
        sum = sum + v[i].x;
        sum = sum + v[i].y;
        sum = sum + v[i].z;
        sum = sum + v[i].w;
    }
}
template <int G>
__device__ __forceinline__ void read_group(float4 (&v)[G], const float4* e4, int g) {
#pragma unroll
    for (int i = 0; i < G; i++) v[i] = e4[g * G + i];
}
// The softmax denominator in one lane: sum = sum + e_j for j = 0..n-1.  The
// caller pads e with -0.0 up to n64 = a multiple of 64; sum + -0.0 == sum for
// every sum (signed zeros and NaN included), so the padding changes no bit.
__device__ __forceinline__ float seq_sum(const float* __restrict__ e, int n64) {
    const float4* e4 = reinterpret_cast<const float4*>(e);
    const int ng = n64 / 64;
    float sum = 0.0f;
    if (ng == 0) return sum;
    float4 a[16], b[16];
    read_group<16>(a, e4, 0);
    for (int g = 0; g < ng; g += 2) {
        read_group<16>(b, e4, g + 1 < ng ? g + 1 : g);  // past the end: a re-read, never added
        __builtin_amdgcn_sched_barrier(0);
        sum_group<16>(sum, a);
        __builtin_amdgcn_sched_barrier(0);
        if (g + 1 >= ng) break;
        read_group<16>(a, e4, g + 2 < ng ? g + 2 : g + 1);
        __builtin_amdgcn_sched_barrier(0);
        sum_group<16>(sum, b);
        __builtin_amdgcn_sched_barrier(0);
    }
    return sum;
}
__host__ __device__ constexpr int pad64(int n) { return (n + 63) & ~63; }

// The same sum for n <= 64 over ceil(n/4) float4 (e padded with -0.0 to a
// multiple of 4), every read issued before the first add.
__device__ __forceinline__ float seq_sum_small(const float* __restrict__ e, int n) {
    const float4* e4 = reinterpret_cast<const float4*>(e);
    const int g = (n + 3) >> 2;
    float4 a[16];
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (i < g) a[i] = e4[i];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (i < g) {
            sum = sum + a[i].x;
            sum = sum + a[i].y;
            sum = sum + a[i].z;
            sum = sum + a[i].w;
        }
    return sum;
}

// ----------------------------------------------------------------------------
// Short contexts (pos < 64, head_dim DT <= 128): one workgroup per query head.
// Every global load is issued at entry, before any is used: the new q/k/v pair
// (and biases, rotation factors) of thread p < DT/2, thread j < pos's k row
// into registers, and the V rows 0..pos-1, so the kernel waits for memory once.
// Then RoPE, the V rows and new rows into LDS, scores, max, exps, the
// sequential softmax sum (lane 0) and the sequential P.V chains (lane d).
// ----------------------------------------------------------------------------
constexpr int kSmallCtx = 64;

template <int DT, typename CT>
__global__ __launch_bounds__(256) void k_attn_small(AttnIn a, RopeTab tab, float* __restrict__ out,
                                                    uint8_t* __restrict__ xq) {
    constexpr int NT = 256, D4 = DT / 4, VU = (kSmallCtx * D4 + NT - 1) / NT;
    __shared__ float4 qs4[D4], ks4[D4], vs4[D4];
    __shared__ float4 V4[kSmallCtx * D4];
    __shared__ __align__(16) float e[kSmallCtx];
    __shared__ float red[NT / 64];
    __shared__ float sh_inv;
    const int tid = threadIdx.x, head = blockIdx.x, kvh = head / a.group, pos = a.pos, n = pos + 1;
    const int64_t ko = (int64_t)kvh * DT;
    const CT* kc = static_cast<const CT*>(a.kc);
    const CT* vc = static_cast<const CT*>(a.vc);
    // the new rows of this head: pair p of q and of k (rotated), element d of v
    const int64_t qo = (int64_t)head * DT;
    const bool pr = tid < DT / 2;
    const int i2 = 2 * (pr ? tid : 0);
    float2 q2 = *reinterpret_cast<const float2*>(a.q + qo + i2);
    float2 k2 = *reinterpret_cast<const float2*>(a.knew + ko + i2);
    float vv = a.vnew[ko + (tid < DT ? tid : 0)];
    float2 bq2 = make_float2(0.0f, 0.0f), bk2 = make_float2(0.0f, 0.0f);
    float bv = 0.0f;
    if (a.bq != nullptr) bq2 = *reinterpret_cast<const float2*>(a.bq + qo + i2);
    if (a.bk != nullptr) bk2 = *reinterpret_cast<const float2*>(a.bk + ko + i2);
    if (a.bv != nullptr) bv = a.bv[ko + (tid < DT ? tid : 0)];
    const float rc = tab.c[pr ? tid : 0], rs = tab.s[pr ? tid : 0];
    float4 kr[D4];
    if (tid < pos) {
        const CT* p = kc + (int64_t)tid * a.row + ko;
#pragma unroll
        for (int i = 0; i < D4; i++) kr[i] = Cache<CT>::ld4(p + 4 * i);
    }
    typename Cache<CT>::Raw vr[VU];
#pragma unroll
    for (int u = 0; u < VU; u++) {
        const int f = tid + u * NT, r = f / D4;
        if (r < pos) vr[u] = Cache<CT>::ldr(vc + (int64_t)r * a.row + ko + 4 * (f % D4));
    }
    float* qs = reinterpret_cast<float*>(qs4);
    float* ks = reinterpret_cast<float*>(ks4);
    float* vs = reinterpret_cast<float*>(vs4);
    // bias, RoPE (bpd_rope_norm_freqs_cpu: pairs below rot turn, the rest pass
    // through), the new rows into LDS; the first query head of each group writes
    // cache row pos; every head takes row pos from its own LDS copy, so no
    // workgroup reads a row another writes
    const bool wr = head % a.group == 0;
    if (pr) {
        float x0 = q2.x, x1 = q2.y, k0 = k2.x, k1 = k2.y;
        if (a.bq != nullptr) {
            x0 = x0 + bq2.x;
            x1 = x1 + bq2.y;
        }
        if (a.bk != nullptr) {
            k0 = k0 + bk2.x;
            k1 = k1 + bk2.y;
        }
        const bool rot = tid < a.rot;
        qs[i2] = rot ? x0 * rc - x1 * rs : x0;
        qs[i2 + 1] = rot ? x0 * rs + x1 * rc : x1;
        const float y0 = rot ? k0 * rc - k1 * rs : k0, y1 = rot ? k0 * rs + k1 * rc : k1;
        ks[i2] = Cache<CT>::rt(y0);
        ks[i2 + 1] = Cache<CT>::rt(y1);
        if (wr) {
            CT* kw = const_cast<CT*>(kc) + (int64_t)pos * a.row + ko;
            Cache<CT>::st(kw + i2, y0);
            Cache<CT>::st(kw + i2 + 1, y1);
        }
    }
    if (tid < DT) {
        if (a.bv != nullptr) vv = vv + bv;
        vs[tid] = Cache<CT>::rt(vv);
        if (wr) Cache<CT>::st(const_cast<CT*>(vc) + (int64_t)pos * a.row + ko + tid, vv);
    }
#pragma unroll
    for (int u = 0; u < VU; u++) {
        const int f = tid + u * NT, r = f / D4;
        if (r < pos) V4[f] = Cache<CT>::cvt(vr[u]);
    }
    __syncthreads();
    float m = -1e38f;
    if (tid < n) {
        const float sc = tid < pos ? dot_regs<D4>(qs4, kr) : dot_ptr(qs4, ks4, D4);
        const float sv = sc * a.scale;
        e[tid] = sv;
        m = sv;
    }
    const float mx = block_max<NT>(m, red);
    if (tid < n)
        e[tid] = expf_libm(e[tid] - mx);
    else if (tid < pad64(n))
        e[tid] = -0.0f;
    __syncthreads();
    if (tid == 0) {
        const float sum = seq_sum_small(e, n);
        sh_inv = sum == 0.0f ? 0.0f : 1.0f / sum;
    }
    __syncthreads();
    if (tid < DT) {
        const float inv = sh_inv;
        const float* Vf = reinterpret_cast<const float*>(V4);
        float acc = 0.0f;
        for (int j = 0; j < pos; j++) acc = acc + Vf[j * DT + tid] * (e[j] * inv);
        acc = acc + vs[tid] * (e[pos] * inv);
        const int64_t o = (int64_t)head * DT + tid;
        out[o] = acc;
        if (xq != nullptr) q8_0_lane_store(acc, xq + (o >> 5) * kQ80Bytes, tid & 31);
    }
}

// ----------------------------------------------------------------------------
// Longer contexts, two kernels.
// k_attn_scores, grid (kv heads * ceil(n/64)), one wave per query head of the
// kv head's group: the workgroup loads k rows 64b .. 64b+63 once, coalesced,
// into LDS (rows at a padded pitch), and lane j of wave h computes
// v_j = (q_h . k_j) * scale, the dot sequential over d, into sc[h][j].  The
// block holding row pos ropes the new k row into its LDS row (the cache row is
// not read) and writes the new k and v rows to the caches, once per kv head.
// ----------------------------------------------------------------------------
constexpr int kScoreRows = 64;
constexpr int kMaxGroup = 8;  // waves per workgroup; larger groups loop over their heads

__host__ __device__ constexpr int score_pitch(int D) { return D + 4; }  // floats: rows 4 banks apart

// Cache rows j0 .. j0+rows-1 (kv head at float offset ko of a row) into LDS at
// kt[r * P4 + i], float4 i of row r.  Each thread issues up to 8 loads before
// its first LDS write: a write right after each load would wait for that load,
// and the rows would arrive one memory latency after another.  Every write
// happens (past the end into `spare`, a float4 of LDS nobody reads): a write
// under a branch lets the compiler sink its load into the branch, behind the
// previous writes.
template <typename CT>
__device__ __forceinline__ void rows_to_lds(float4* kt, float4* spare, const CT* kc, int j0, int rows, int64_t row,
                                            int64_t ko, int D4, int P4) {
    constexpr int B = 8;
    const int n = rows * D4;
    for (int f0 = threadIdx.x; f0 < n; f0 += B * (int)blockDim.x) {
        typename Cache<CT>::Raw t[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int f = min(f0 + u * (int)blockDim.x, n - 1);  // past the end: a re-read, never stored
            t[u] = Cache<CT>::ldr(kc + (int64_t)(j0 + f / D4) * row + ko + 4 * (f % D4));
        }
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int f = f0 + u * (int)blockDim.x;
            float4* dst = f < n ? kt + (f / D4) * P4 + f % D4 : spare;
            *dst = Cache<CT>::cvt(t[u]);
        }
    }
}

template <int DT, typename CT>
__global__ __launch_bounds__(64 * kMaxGroup) void k_attn_scores(AttnIn a, RopeTab tab, float* __restrict__ sc, int ld) {
    extern __shared__ float4 sm4[];
    const int D = DT > 0 ? DT : a.D, D4 = D / 4, P4 = score_pitch(D) / 4, G = a.group;
    const int pos = a.pos, nb = (pos + kScoreRows) / kScoreRows;
    const int kvh = blockIdx.x / nb, yb = blockIdx.x % nb, j0 = yb * kScoreRows;
    const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float4* kt = sm4;                        // [64][P4] the block's k rows
    float4* qs4 = kt + kScoreRows * P4;      // [G][D4] q of the group's heads
    float4* ks4 = qs4 + G * D4;              // the new k row
    float4* vs4 = ks4 + D4;                  // the new v row
    float4* spare = vs4 + D4;                // writes past the tile
    const bool last = yb == nb - 1;          // the block holding row pos
    const int64_t ko = (int64_t)kvh * D;
    // bias + RoPE of the group's q heads in one pass; the q loads of a thread's
    // first pair go out before the k tile's, so both arrive in one memory round trip
    float* qs = reinterpret_cast<float*>(qs4);
    const int half = D / 2;
    const int pp0 = threadIdx.x;
    float2 q0 = make_float2(0.0f, 0.0f);
    if (pp0 < G * half) q0 = *reinterpret_cast<const float2*>(a.q + (int64_t)(kvh * G + pp0 / half) * D + 2 * (pp0 % half));
    // k rows j0 .. min(j0+63, pos-1): float4 i of row r at kt[r*P4 + i]
    const int rows = min(kScoreRows, pos - j0);
    rows_to_lds<CT>(kt, spare, static_cast<const CT*>(a.kc), j0, rows, a.row, ko, D4, P4);
    for (int pp = pp0; pp < G * half; pp += blockDim.x) {
        const int h = pp / half, pr = pp % half, i = 2 * pr;
        const int64_t qo = (int64_t)(kvh * G + h) * D + i;
        float x0, x1;
        if (pp == pp0) {
            x0 = q0.x;
            x1 = q0.y;
        } else {
            x0 = a.q[qo];
            x1 = a.q[qo + 1];
        }
        if (a.bq != nullptr) {
            x0 = x0 + a.bq[qo];
            x1 = x1 + a.bq[qo + 1];
        }
        const float c = tab.c[pr], sn = tab.s[pr];
        const bool rot = pr < a.rot;
        qs[h * D + i] = rot ? x0 * c - x1 * sn : x0;
        qs[h * D + i + 1] = rot ? x0 * sn + x1 * c : x1;
    }
    // the block holding row pos also writes the new k and v rows to the caches
    if (last)
        rope_rows<CT>(a, tab, kvh * G, kvh, nullptr, reinterpret_cast<float*>(ks4), reinterpret_cast<float*>(vs4),
                      true, true);
    __syncthreads();
    const int j = j0 + lane;
    if (j > pos) return;
    const float4* kr = j == pos ? ks4 : kt + lane * P4;
    for (int h = wave; h < G; h += nw) {
        const float4* q = qs4 + h * D4;
        float s = 0.0f;
        if (DT > 0) {
#pragma unroll 8
            for (int i = 0; i < DT / 4; i++) s = dot_step(s, q[i], kr[i]);
        } else {
            for (int i = 0; i < D4; i++) s = dot_step(s, q[i], kr[i]);
        }
        sc[(int64_t)(kvh * G + h) * ld + j] = s * a.scale;
    }
}

// k_attn_pv, grid (heads * head_dim/COLS, query tokens): softmax and P.V for COLS
// output columns d0..d0+COLS-1 of one head, in the reference's order.  The scores go to LDS; max,
// exps and the weights w_j = e_j * inv are parallel; the softmax sum runs in
// lane 0 and each output's chain acc = RN(acc + RN(v_jd * w_j)) in lane d - d0
// of wave 0.  Wave 0 does nothing else during P.V: waves 1-4 (the producers)
// stream the V columns through a two-slot LDS ring of ROWS-row chunks.  Every
// producer keeps the loads of the next AHEAD chunks in flight in registers and
// writes one chunk of products per step, transposed so that column d of a
// chunk is one padded LDS row; one barrier per chunk.  Rows past n get -0.0,
// which leaves the chain unchanged (acc + -0.0 == acc), so every chunk is read
// as whole float4.
// ----------------------------------------------------------------------------
constexpr int kPvProd = 256;               // producer threads
constexpr int kPvThreads = 64 + kPvProd;   // wave 0 runs the chains
constexpr int kPvBigMin = 1024;            // 128-row chunks from here ...
constexpr int kPvBigMax = 16384;           // ... up to here (LDS: ring + scores)

// COLS 16 leaves twice as many workgroups each streaming half the V bytes (the
// stream is bound by the bytes each workgroup keeps in flight); 32 when the
// outputs' Q8_0 blocks (32 columns) are written too.  With a 132-float pitch
// the producers' transposed writes hit 64 distinct banks at COLS 16.
template <int ROWS, int COLS>
struct PvShape {
    static constexpr int C4 = COLS / 4;              // float4 of a V row slice
    static constexpr int LD = ROWS + 4;              // ring row pitch in floats
    static constexpr int PER = ROWS * C4 / kPvProd;  // float4 of a chunk per producer
    static constexpr int AHEAD = 4096 / (ROWS * C4) < 8 ? 4096 / (ROWS * C4) : 8;  // chunks in flight (<= 64 KB)
};
// LDS: the ring, the padded scores and a few words
static_assert(kMaxCtx % 64 == 0 && 2 * 32 * PvShape<64, 32>::LD * 4 + kMaxCtx * 4 + 256 + 64 <= 160 * 1024,
              "k_attn_pv<64> LDS");
static_assert(kPvBigMax % 64 == 0 && 2 * 32 * PvShape<128, 32>::LD * 4 + kPvBigMax * 4 + 256 + 64 <= 160 * 1024,
              "k_attn_pv<128> LDS");

template <typename CT>
struct PvPipe {
    const CT* vbase;     // V column d0 of the head's kv row 0
    int row, n, nch, tid;  // tid: producer number, or the chain lane
    const float* e;      // exps in LDS
    float inv;
};

// Load of chunk c's share of producer tid: float4 number f = tid + k*256 is
// row c*ROWS + f/C4, columns d0 + 4(f%C4)..+3; rows past n repeat row n-1 (never
// used, so every load stays in the cache rows already written).
template <int ROWS, int COLS, typename CT>
__device__ __forceinline__ typename Cache<CT>::Raw pv_load(const PvPipe<CT>& p, int c, int k) {
    constexpr int C4 = COLS / 4;
    const int f = p.tid + k * kPvProd, r = min(c * ROWS + f / C4, p.n - 1);
    return Cache<CT>::ldr(p.vbase + (int64_t)r * p.row + 4 * (f % C4));
}

// Step c = c0 + U (pf slot U holds chunk c; U is a template argument so that pf
// is indexed by constants only): the producers write chunk c's products to
// ring slot c&1 and refill with chunk c + AHEAD; barrier; the chain lanes add
// the chunk's ROWS products in row order.  Slot c&1 is written again at step
// c+2, after the barrier of step c+1, which the chain reaches only once it has
// added chunk c.
template <int U, int ROWS, int COLS, typename CT>
__device__ __forceinline__ void pv_chunk(
    const PvPipe<CT>& p, bool prod, bool chain,
    typename Cache<CT>::Raw (&pf)[PvShape<ROWS, COLS>::AHEAD * PvShape<ROWS, COLS>::PER], float* ring, int c0,
    float& acc) {
    using PS = PvShape<ROWS, COLS>;
    constexpr int PER = PS::PER, LD = PS::LD, C4 = PS::C4;
    const int c = c0 + U;
    if (c >= p.nch) return;  // uniform over the workgroup
    float* slot = ring + (c & 1) * COLS * LD;
    if (prod) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int f = p.tid + k * kPvProd, rr = f / C4, r = c * ROWS + rr;
            const float4 v = Cache<CT>::cvt(pf[U * PER + k]);
            float* dst = slot + 4 * (f % C4) * LD + rr;
            if (r < p.n) {
                const float w = p.e[r] * p.inv;  // the reference's scores[j] *= inv_sum
                dst[0] = v.x * w;
                dst[LD] = v.y * w;
                dst[2 * LD] = v.z * w;
                dst[3 * LD] = v.w * w;
            } else {
                dst[0] = -0.0f;
                dst[LD] = -0.0f;
                dst[2 * LD] = -0.0f;
                dst[3 * LD] = -0.0f;
            }
            pf[U * PER + k] = pv_load<ROWS, COLS, CT>(p, c + PS::AHEAD, k);
        }
    }
    __syncthreads();
    if (chain) {
        // the chunk's products as 16-float4 groups (sum_group), the second
        // group's reads issued before the first group's adds
        const float4* col = reinterpret_cast<const float4*>(slot + p.tid * LD);
        static_assert(ROWS == 64 || ROWS == 128, "one or two 16-float4 groups per chunk");
        float4 a[16], b[16];
        read_group<16>(a, col, 0);
        if constexpr (ROWS == 128) read_group<16>(b, col, 1);
        __builtin_amdgcn_sched_barrier(0);
        sum_group<16>(acc, a);
        if constexpr (ROWS == 128) {
            __builtin_amdgcn_sched_barrier(0);
            sum_group<16>(acc, b);
        }
    }
}

// Workgroup b's head and column slice.  Workgroups go to the 8 XCDs round robin
// (b % 8), each with its own L2: when the (kv head, slice) pairs divide into 8,
// the `group` heads that read one V slice get workgroups of one XCD, so the
// slice comes from HBM once per group instead of once per head.
__device__ __forceinline__ void pv_tile(int b, int H, int group, int slices, int& head, int& slice) {
    const int hkv = H / group;
    if ((hkv * slices) % 8 == 0) {
        const int i = b >> 3, pair = (i / group) * 8 + (b & 7);
        head = (pair % hkv) * group + i % group;
        slice = pair / hkv;
    } else {
        head = b % H;
        slice = b / H;
    }
}

template <int ROWS, int COLS, typename CT>
__global__ __launch_bounds__(kPvThreads) void k_attn_pv(AttnIn a, const float* __restrict__ sc, int ld,
                                                        float* __restrict__ out, uint8_t* __restrict__ xq) {
    using PS = PvShape<ROWS, COLS>;
    constexpr int NT = kPvThreads, PER = PS::PER, AHEAD = PS::AHEAD;
    static_assert(AHEAD == 4 || AHEAD == 8, "one pv_chunk call per chunk in flight");
    static_assert(COLS == 16 || COLS == 32, "16 or 32 chain lanes (32: the outputs' Q8_0 blocks)");
    extern __shared__ float4 e4dyn[];
    float* e = reinterpret_cast<float*>(e4dyn);  // pad64(n) floats
    __shared__ __align__(16) float ring[2 * COLS * PS::LD];
    __shared__ uint64_t etab[32];
    __shared__ float red[NT / 64];
    __shared__ float sh_inv;
    const int H = a.row / a.D * a.group;
    int head, slice;
    pv_tile(blockIdx.x, H, a.group, a.D / COLS, head, slice);
    const int d0 = COLS * slice;
    // query token blockIdx.y of a batch: its position is a.pos + blockIdx.y, its
    // scores and outputs follow the previous token's
    const int tq = blockIdx.y;
    sc += (int64_t)tq * H * ld;
    out += (int64_t)tq * H * a.D;
    if (xq != nullptr) xq += (int64_t)tq * (H * a.D / 32) * kQ80Bytes;
    const int tid = threadIdx.x, kvh = head / a.group, n = a.pos + tq + 1, nch = (n + ROWS - 1) / ROWS;
    const bool prod = tid >= 64, chain = tid < COLS;
    if (tid < 32) etab[tid] = kExp2fTab[tid];  // published by block_max's barrier
    // the scores first, 8 loads in flight (loads complete in order, so anything
    // issued before them would be waited for too), then the first V chunks,
    // which stream in while the softmax runs
    float m = -1e38f;
    const float* scr = sc + (int64_t)head * ld;
    for (int j0 = tid; j0 < n; j0 += 8 * NT) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = scr[min(j0 + u * NT, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * NT;
            if (j < n) {
                e[j] = t[u];
                m = t[u] > m ? t[u] : m;
            }
        }
    }
    PvPipe<CT> pp{static_cast<const CT*>(a.vc) + (int64_t)kvh * a.D + d0, a.row, n, nch, prod ? tid - 64 : tid, e,
                  0.0f};
    typename Cache<CT>::Raw pf[AHEAD * PER];
    if (prod) {
#pragma unroll
        for (int c = 0; c < AHEAD; c++)
#pragma unroll
            for (int k = 0; k < PER; k++) pf[c * PER + k] = pv_load<ROWS, COLS, CT>(pp, c, k);
    }
    const float mx = block_max<NT>(m, red);
    // the exps with the table in LDS (a per-lane index into constant memory is a
    // load from the cache hierarchy per call)
    const int n64 = pad64(n);
    for (int j = tid; j < n64; j += NT) e[j] = j < n ? expf_libm(e[j] - mx, etab) : -0.0f;
    __syncthreads();
    if (tid == 0) {
        const float sum = seq_sum(e, n64);
        sh_inv = sum == 0.0f ? 0.0f : 1.0f / sum;
    }
    __syncthreads();
    pp.inv = sh_inv;
    float acc = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += AHEAD) {
        pv_chunk<0, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
        pv_chunk<1, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
        pv_chunk<2, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
        pv_chunk<3, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
        if constexpr (AHEAD == 8) {
            pv_chunk<4, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
            pv_chunk<5, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
            pv_chunk<6, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
            pv_chunk<7, ROWS, COLS, CT>(pp, prod, chain, pf, ring, c0, acc);
        }
    }
    if (chain) {
        const int64_t o = (int64_t)head * a.D + d0 + tid;
        out[o] = acc;
        if constexpr (COLS == 32)
            if (xq != nullptr) q8_0_lane_store(acc, xq + (o >> 5) * kQ80Bytes, tid & 31);
    }
}

// ----------------------------------------------------------------------------
// SwiGLU (bpd_swiglu_fuse_cpu, bench/bpd_cpu.c:5504-5507):
//   y = (g / (1 + expf(-g))) * u, written over gate, and Q8_0(y).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_swiglu(float* gate, const float* __restrict__ up, uint8_t* __restrict__ xq,
                                                int F) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= F) return;  // F % 32 == 0: whole Q8_0 blocks leave together
    const float g = gate[i];
    const float y = (g / (1.0f + expf_libm(-g))) * up[i];
    gate[i] = y;
    if (xq != nullptr) q8_0_lane_store(y, xq + (int64_t)(i >> 5) * kQ80Bytes, i & 31);
}

// ----------------------------------------------------------------------------
// Argmax (bpd_argmax_dim_cpu, bench/bpd_cpu.c:4512-4526): best = x[0], then
// x[k] replaces it when x[k] > best.  So the result is the first index of the
// largest non-NaN value (+0 and -0 tie), or 0 when x[0] is NaN.
// ----------------------------------------------------------------------------
__device__ __forceinline__ bool argmax_beats(float b, int bi, float a, int ai) {
    if (bi == INT_MAX) return false;
    if (ai == INT_MAX) return true;
    return b > a || (b == a && bi < ai);
}

__device__ __forceinline__ void argmax_take(float v, int i, float& best, int& idx) {
    if (v == v && (idx == INT_MAX || v > best)) {
        best = v;
        idx = i;
    }
}

// Each thread scans float4 chunks t, t + NT, ... (8 loads in flight), then the
// n % 4 tail, so it meets its indices in increasing order and keeps the first
// of equal values; lanes and waves then combine by (value, lower index).
// Workgroup b takes row b of [rows][n] and writes out[b] (int32) or, with out
// NULL, out64[b] (the reference's long, bpd_argmax_dim_cpu with outer = rows).
// Rows after the first are read as float4 only when n % 4 == 0 (16-byte
// aligned); otherwise element by element.
template <int NT>
__global__ __launch_bounds__(NT) void k_argmax(const float* __restrict__ x, int n, int32_t* __restrict__ out,
                                               int64_t* __restrict__ out64) {
    __shared__ float bv[NT / 64];
    __shared__ int bi[NT / 64];
    x += (int64_t)blockIdx.x * n;
    const bool vec = blockIdx.x == 0 || (n & 3) == 0;
    const int tid = threadIdx.x, nc = vec ? n >> 2 : 0;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float best = 0.0f;
    int idx = INT_MAX;  // no candidate yet
    for (int c0 = tid; c0 < nc; c0 += 8 * NT) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int c = c0 + u * NT;
            v[u] = c < nc ? x4[c] : make_float4(__builtin_nanf(""), 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int c = c0 + u * NT;
            if (c < nc) {
                argmax_take(v[u].x, 4 * c, best, idx);
                argmax_take(v[u].y, 4 * c + 1, best, idx);
                argmax_take(v[u].z, 4 * c + 2, best, idx);
                argmax_take(v[u].w, 4 * c + 3, best, idx);
            }
        }
    }
    for (int i = 4 * nc + tid; i < n; i += NT) argmax_take(x[i], i, best, idx);
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        const float ob = xor_f(best, mask);
        const int oi = xor_i(idx, mask);
        if (argmax_beats(ob, oi, best, idx)) {
            best = ob;
            idx = oi;
        }
    }
    if ((tid & 63) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NT / 64; w++)
            if (argmax_beats(bv[w], bi[w], best, idx)) {
                best = bv[w];
                idx = bi[w];
            }
        const float x0 = x[0];
        const int r = (!(x0 == x0) || idx == INT_MAX) ? 0 : idx;
        if (out != nullptr)
            out[blockIdx.x] = r;
        else
            out64[blockIdx.x] = r;
    }
}

// ----------------------------------------------------------------------------
// fp32 head y[N] = W[N][K] h (the reference driver's weight-tied fallback,
// inference/llamatov_c_inference.py:179-186; its library has no source).
// Order: lane l sums W[r][l + 64 i] * h[l + 64 i] over i from +0.0, then the
// lanes combine by xor-32, 16, 8, 4, 2, 1 steps (p_l = p_l + p_{l^m}).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ W, const float* __restrict__ x,
                                                  float* __restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= N) return;
    const float* wr = W + (int64_t)r * K;
    float acc = 0.0f;
    for (int k = lane; k < K; k += 64) acc = acc + wr[k] * x[k];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + xor_f(acc, m);
    if (lane == 0) y[r] = acc;
}

__global__ __launch_bounds__(256) void k_expf(const float* __restrict__ x, float* __restrict__ y, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = expf_libm(x[i]);
}

// ----------------------------------------------------------------------------
// Several tokens through the block (bpd_llama_block_cpu with n_tokens > 1): the
// reference ropes q and k of every token (bpd_rope_norm_freqs_cpu,
// bench/bpd_cpu.c:5146-5184) and writes every k and v row to the caches
// (:5204-5260) before attention reads them, so the batch takes three kernels:
// k_rope_write, k_mt_scores, then k_attn_pv with one grid row per token.
// ----------------------------------------------------------------------------
// The rotation of token t, pair j: cos and sin of pos_ids[t] * theta_scale^j /
// rope_freqs[j] (host libm), pairs j < rot.
struct RopeCS {
    float c, s;
};

// Workgroup t: q of token t (H heads of D, in place), k (roped) and v of its
// kv heads to cache row pos[t].
template <typename CT>
__global__ __launch_bounds__(256) void k_rope_write(float* __restrict__ q, const float* __restrict__ k,
                                                    const float* __restrict__ v, CT* __restrict__ kc,
                                                    CT* __restrict__ vc, const int32_t* __restrict__ pos,
                                                    const RopeCS* __restrict__ tab, int H, int HKV, int D, int rot) {
    const int t = blockIdx.x, half = D / 2, row = HKV * D;
    const RopeCS* tt = tab + (int64_t)t * (kMaxHeadDim / 2);
    float* qt = q + (int64_t)t * H * D;
    for (int pp = threadIdx.x; pp < H * half; pp += blockDim.x) {
        const int p = pp % half, i = 2 * (pp / half) * half + 2 * p;
        if (p >= rot) continue;
        const float x0 = qt[i], x1 = qt[i + 1], c = tt[p].c, sn = tt[p].s;
        qt[i] = x0 * c - x1 * sn;
        qt[i + 1] = x0 * sn + x1 * c;
    }
    const int64_t ro = (int64_t)t * row, co = (int64_t)pos[t] * row;
    for (int pp = threadIdx.x; pp < HKV * half; pp += blockDim.x) {
        const int p = pp % half, i = 2 * pp;
        float y0 = k[ro + i], y1 = k[ro + i + 1];
        if (p < rot) {
            const float x0 = y0, x1 = y1, c = tt[p].c, sn = tt[p].s;
            y0 = x0 * c - x1 * sn;
            y1 = x0 * sn + x1 * c;
        }
        Cache<CT>::st(kc + co + i, y0);
        Cache<CT>::st(kc + co + i + 1, y1);
    }
    for (int d = threadIdx.x; d < row; d += blockDim.x) Cache<CT>::st(vc + co + d, v[ro + d]);
}

// Scores of the batch, grid (row blocks, kv heads, tokens): workgroup (b, kvh,
// t) loads cache k rows 64b..64b+63 (those <= kv_pos + t, the token's causal
// limit) once into LDS, and lane j of wave h computes row j's score for query
// head kvh * G + h of token t: s = sum_d q_d k_d sequentially over d, times
// scale, into sc[t][head][j].
template <typename CT>
__global__ __launch_bounds__(64 * kMaxGroup) void k_mt_scores(const float* __restrict__ q, const CT* __restrict__ kc,
                                                              float* __restrict__ sc, int ld, int kv_pos, int H,
                                                              int HKV, int D, float scale) {
    extern __shared__ float4 sm4[];
    const int G = H / HKV, D4 = D / 4, P4 = score_pitch(D) / 4, row = HKV * D;
    const int j0 = blockIdx.x * kScoreRows, kvh = blockIdx.y, t = blockIdx.z, qpos = kv_pos + t;
    if (j0 > qpos) return;  // uniform over the workgroup
    const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float4* kt = sm4;                    // [64][P4]
    float4* qs4 = kt + kScoreRows * P4;  // [G][D4]
    float4* spare = qs4 + G * D4;        // writes past the tile
    const int rows = min(kScoreRows, qpos + 1 - j0);
    const int64_t ko = (int64_t)kvh * D;
    rows_to_lds<CT>(kt, spare, kc, j0, rows, row, ko, D4, P4);
    const float4* qt = reinterpret_cast<const float4*>(q + ((int64_t)t * H + kvh * G) * D);
    for (int f = threadIdx.x; f < G * D4; f += blockDim.x) qs4[f] = qt[f];
    __syncthreads();
    if (lane >= rows) return;
    const float4* kr = kt + lane * P4;
    for (int h = wave; h < G; h += nw) {
        const float4* qh = qs4 + h * D4;
        float s = 0.0f;
#pragma unroll 8
        for (int i = 0; i < D4; i++) s = dot_step(s, qh[i], kr[i]);
        sc[((int64_t)t * H + kvh * G + h) * ld + j0 + lane] = s * scale;
    }
}

// ----------------------------------------------------------------------------
// Attention of a batch of T tokens laid out for throughput: the arithmetic of
// k_mt_scores + k_attn_pv (the reference's per-token order), with query token t
// attending over rows 0..n_t-1, n_t = kv_pos + t + 1.  Those kernels give each
// (head, token) a workgroup whose chains run in one lane (the softmax sum) or 32
// (P.V); at T = 512 that is 65,536 workgroups of mostly idle lanes.  Here a
// wave-instruction advances many tokens' chains:
//   k_mt_scores_tile  grid (64-row blocks, kv heads, 16-token blocks): k rows and
//                     the block's q rows in LDS; lane j of a wave runs TPW tokens'
//                     dots with row j (sequential over d, TPW chains per lane).
//   k_mt_softmax      grid (heads, 64-token blocks), 8 waves: each thread's score
//                     quads in registers, the order-free max, e = expf(v - m) into
//                     LDS, lane t of wave 0 adds token t's e in row order, then the
//                     weights w = RN(e * inv), inv = S == 0 ? 0 : 1/S, over the scores.
//   k_mt_pv           grid (heads, 64-token block pairs, 64-column slices): per 64-row
//                     chunk the weights (transposed) and the V rows in LDS; lane
//                     (tg, cg) runs 4 tokens x 4 columns of chains
//                     acc = RN(acc + RN(v*w)) in row order, then Q8_0(out).
// Score rows are ld floats apart, ld a multiple of 64 (16-byte aligned rows).
// ----------------------------------------------------------------------------
constexpr int kMtTok = 16;  // tokens per scores workgroup
constexpr int kMtBlk = 64;  // tokens per softmax / P.V workgroup (one per lane)

__host__ __device__ constexpr size_t mt_scores_lds(int G, int D) {
    return ((size_t)kScoreRows * score_pitch(D) + (size_t)kMtTok * G * D + 4) * 4;
}

// 8 waves in REPS = 16 / TPW token subsets: with REPS > 1 (the host keeps
// G * REPS <= 8) wave w takes head w % G of the kv head's group and tokens
// TPW(w / G) .. +TPW-1 of the block; with REPS = 1 wave w takes heads w, w + 8, ...
// and all 16 tokens.
template <typename CT, int TPW>
__global__ __launch_bounds__(64 * kMaxGroup) void k_mt_scores_tile(const float* __restrict__ q,
                                                                   const CT* __restrict__ kc, float* __restrict__ sc,
                                                                   int ld, int kv_pos, int T, int H, int HKV, int D,
                                                                   float scale) {
    static_assert(kMtTok % TPW == 0, "token subsets of the block");
    extern __shared__ float4 sm4[];
    const int G = H / HKV, D4 = D / 4, P4 = score_pitch(D) / 4, row = HKV * D;
    const int j0 = blockIdx.x * kScoreRows, kvh = blockIdx.y, t0 = blockIdx.z * kMtTok;
    const int nt = min(kMtTok, T - t0), n_hi = kv_pos + t0 + nt;  // rows of the block's last token
    if (j0 >= n_hi) return;  // uniform over the workgroup
    const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float4* kt = sm4;                    // [64][P4]
    float4* qs4 = kt + kScoreRows * P4;  // [kMtTok][G][D4]
    float4* spare = qs4 + kMtTok * G * D4;
    const int rows = min(kScoreRows, n_hi - j0);
    rows_to_lds<CT>(kt, spare, kc, j0, rows, row, (int64_t)kvh * D, D4, P4);
    // the block's q rows, 4 loads in flight per thread before any LDS write (every
    // write happens, past the end into `spare`, so no load sinks into a branch)
    const int nq = kMtTok * G * D4;
    for (int f0 = threadIdx.x; f0 < nq; f0 += 4 * (int)blockDim.x) {
        float4 t[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = min(f0 + u * (int)blockDim.x, nq - 1), tt = f / (G * D4), r = f % (G * D4);
            t[u] = tt < nt ? reinterpret_cast<const float4*>(q + ((int64_t)(t0 + tt) * H + kvh * G) * D)[r]
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = f0 + u * (int)blockDim.x;
            *(f < nq ? qs4 + f : spare) = t[u];
        }
    }
    __syncthreads();
    if (lane >= rows) return;
    const float4* kr = kt + lane * P4;
    constexpr int REPS = kMtTok / TPW;
    const int sub = REPS == 1 ? 0 : wave / G, ts0 = TPW * sub;
    if (sub >= REPS) return;
    for (int h = REPS == 1 ? wave : wave % G; h < G; h += REPS == 1 ? nw : G) {
        float s[TPW];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++) s[tt] = 0.0f;
        for (int i = 0; i < D4; i++) {
            const float4 k4 = kr[i];
#pragma unroll
            for (int tt = 0; tt < TPW; tt++) s[tt] = dot_step(s[tt], qs4[((ts0 + tt) * G + h) * D4 + i], k4);
        }
#pragma unroll
        for (int tt = 0; tt < TPW; tt++)
            if (ts0 + tt < nt) sc[((int64_t)(t0 + ts0 + tt) * H + kvh * G + h) * ld + j0 + lane] = s[tt] * scale;
    }
}

constexpr int kMtSmThreads = 512;  // thread p: row quad p % 16 of tokens p / 16 and p / 16 + 32
constexpr int kMtSmGroup = 8;      // 64-row chunks of e in LDS at once

// LDS pitch of a token's e rows in k_mt_softmax: a group of up to kMtSmGroup
// chunks plus 4 floats, so the chain lanes' float4 reads (one token each, rows
// 4 banks apart) are conflict-free.
__host__ __device__ constexpr int mt_sm_pitch(int nch) {
    return kScoreRows * (nch < kMtSmGroup ? nch : kMtSmGroup) + 4;
}
__host__ __device__ constexpr size_t mt_sm_lds(int nch) { return (size_t)kMtBlk * mt_sm_pitch(nch) * 4; }

// The chunks g0 .. g0+kMtSmGroup-1 of one token row (float4 jq of each; rows
// past the last chunk are not read).  Every load is issued before any is used.
__device__ __forceinline__ void mt_sm_load(float4 (&v)[kMtSmGroup], const float* row, bool has, int g0, int nch) {
#pragma unroll
    for (int c = 0; c < kMtSmGroup; c++)
        v[c] = has && g0 + c < nch ? *reinterpret_cast<const float4*>(row + kScoreRows * (g0 + c))
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

template <int NT>
__global__ __launch_bounds__(NT) void k_mt_softmax(float* __restrict__ sc, int ld, int kv_pos, int T, int H) {
    static_assert(NT == 512 && kMtBlk == 64, "16 threads per token row, two tokens per thread");
    extern __shared__ float4 sm_e4[];
    float* E = reinterpret_cast<float*>(sm_e4);  // [token][EP]: e of the group's rows, +0.0 past the token's
    __shared__ uint64_t etab[32];
    __shared__ float inv_s[kMtBlk];
    const int h = blockIdx.x, tb = blockIdx.y * kMtBlk, p = threadIdx.x, jq = p & 15, lane = p & 63;
    const int nt = min(kMtBlk, T - tb), n_hi = kv_pos + tb + nt, nch = (n_hi + kScoreRows - 1) / kScoreRows;
    const int ng = (nch + kMtSmGroup - 1) / kMtSmGroup, EP = mt_sm_pitch(nch);
    if (p < 32) etab[p] = kExp2fTab[p];
    int tt[2], nrow[2];
    bool has[2];
    float* row[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        tt[k] = (p >> 4) + 32 * k;
        has[k] = tt[k] < nt;
        nrow[k] = kv_pos + tb + tt[k] + 1;  // rows of the token
        row[k] = sc + ((int64_t)(tb + (has[k] ? tt[k] : 0)) * H + h) * ld + 4 * jq;
    }
    // the max of each token's row (order-free: every candidate is compared with >
    // and NaN never wins), over the thread's quads, then the token's 16 lanes
    float4 v[2][kMtSmGroup];
    float m[2] = {-1e38f, -1e38f};
    for (int g = 0; g < ng; g++) {
#pragma unroll
        for (int k = 0; k < 2; k++) mt_sm_load(v[k], row[k], has[k], kMtSmGroup * g, nch);
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int c = 0; c < kMtSmGroup; c++) {
                const int j = kScoreRows * (kMtSmGroup * g + c) + 4 * jq;
                const float x[4] = {v[k][c].x, v[k][c].y, v[k][c].z, v[k][c].w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (j + i < nrow[k] && has[k]) m[k] = x[i] > m[k] ? x[i] : m[k];
            }
    }
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) {
            const float y = __shfl_xor(m[k], o, 16);
            m[k] = y > m[k] ? y : m[k];
        }
    __syncthreads();  // etab
    float sum = 0.0f;  // lane t of wave 0: token t's chain
    for (int g = 0; g < ng; g++) {
        if (g > 0) __syncthreads();  // the chain has read the previous group
        if (ng > 1) {  // one group: the registers still hold it
#pragma unroll
            for (int k = 0; k < 2; k++) mt_sm_load(v[k], row[k], has[k], kMtSmGroup * g, nch);
        }
        // e = expf(v - m) over the scores in place, and into LDS; past the token's rows
        // expf(-Inf) = +0.0, which leaves the chain unchanged (it starts at +0.0 and adds
        // only values >= +0.0, so it is never -0.0)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if (!has[k]) continue;
#pragma unroll
            for (int c = 0; c < kMtSmGroup; c++) {
                const int cc = kMtSmGroup * g + c, j = kScoreRows * cc + 4 * jq;
                if (cc >= nch) break;
                const float x[4] = {v[k][c].x, v[k][c].y, v[k][c].z, v[k][c].w};
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; i++) e[i] = expf_libm(j + i < nrow[k] ? x[i] - m[k] : -INFINITY, etab);
                v[k][c] = make_float4(e[0], e[1], e[2], e[3]);
                if (ng > 1) {  // kept for the weights pass
                    float* dst = row[k] + kScoreRows * cc;
                    if (j + 3 < nrow[k]) {
                        *reinterpret_cast<float4*>(dst) = v[k][c];
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (j + i < nrow[k]) dst[i] = e[i];
                    }
                }
                *reinterpret_cast<float4*>(E + tt[k] * EP + kScoreRows * c + 4 * jq) = v[k][c];
            }
        }
        __syncthreads();
        if (p < 64) {
            // token lane's chain over the group's rows in order, one chunk's 16 float4
            // read ahead of the adds
            const float4* col = reinterpret_cast<const float4*>(E + lane * EP);
            const int gc = min(kMtSmGroup, nch - kMtSmGroup * g);
            float4 a[16], b[16];
            read_group<16>(a, col, 0);
            for (int c = 0; c < gc; c += 2) {
                read_group<16>(b, col, c + 1 < gc ? c + 1 : c);  // past the group: a re-read, never added
                __builtin_amdgcn_sched_barrier(0);
                sum_group<16>(sum, a);
                __builtin_amdgcn_sched_barrier(0);
                if (c + 1 >= gc) break;
                read_group<16>(a, col, c + 2 < gc ? c + 2 : c + 1);
                __builtin_amdgcn_sched_barrier(0);
                sum_group<16>(sum, b);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (p < 64) inv_s[p] = sum == 0.0f ? 0.0f : 1.0f / sum;
    __syncthreads();  // also orders each thread's e stores before its reloads
    // the weights w = RN(e * inv) over the scores (the reference's scores[j] *=
    // inv_sum), for the token's rows only
#pragma unroll
    for (int k = 0; k < 2; k++) {
        if (!has[k]) continue;
        const float inv = inv_s[tt[k]];
        for (int g = 0; g < ng; g++) {
            if (ng > 1) mt_sm_load(v[k], row[k], true, kMtSmGroup * g, nch);
#pragma unroll
            for (int c = 0; c < kMtSmGroup; c++) {
                const int cc = kMtSmGroup * g + c, j = kScoreRows * cc + 4 * jq;
                if (cc >= nch) break;
                const float4 w = make_float4(v[k][c].x * inv, v[k][c].y * inv, v[k][c].z * inv, v[k][c].w * inv);
                float* dst = row[k] + kScoreRows * cc;
                if (j + 3 < nrow[k]) {
                    *reinterpret_cast<float4*>(dst) = w;
                } else {
                    const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (j + i < nrow[k]) dst[i] = wv[i];
                }
            }
        }
    }
}

// k_mt_pv: grid (heads, token-block pairs, 64-column slices), 8 waves.  Token
// block i of a causal batch has i + 1 chunks of 64 rows, so workgroup p takes
// block nb - 1 - p and then block p (once when they are the same): every
// workgroup carries nb + 1 chunks of work.  Each wave holds 16 tokens x 32
// columns of the block: lane (tg, cg) = (lane / 16, lane % 16) holds tokens
// 4tg..4tg+3 x columns 2cg, 2cg+1, 8 chains acc = RN(acc + RN(v * w)) in row
// order.  Per row a lane reads a float2 of V (its 2 columns) and a float4 of the
// transposed weights (its 4 tokens).  Chunks of 64 rows are staged in two LDS
// slots (chunk c + 1 written while c is added): the weights the softmax left over
// the scores, transposed to [row][token], and the V rows converted to fp32.  Rows
// past a token's count are skipped by a select, never added.  (One wave carries
// at most half the VALU issue of its SIMD on this loop, so a block's chains are
// spread over all 8 waves, and pairing a heavy block with a light one keeps the
// work per workgroup even.)
constexpr int kPvTok = 64;   // tokens per block
constexpr int kPvCols = 64;  // columns per workgroup
constexpr int kPvThreads2 = 512;

template <typename CT>
struct MtPvStage {
    float4 w[2];                   // float4 f = tid + 512k: token f % 64, rows 4(f / 64)..+3
    typename Cache<CT>::Raw v[2];  // float4 f: row f / 16, columns 4(f % 16)..+3
};

template <typename CT>
__device__ __forceinline__ void mt_pv_load(MtPvStage<CT>& st, const float* __restrict__ wsc, const CT* __restrict__ vbase,
                                           int j0, int tb, int nt, int h, int H, int ld, int n_hi, int row, int ncol) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
        // consecutive lanes take consecutive tokens, so the transposed LDS writes
        // of a wave hit 64 different banks
        const int f = (int)threadIdx.x + kPvThreads2 * k, tt = min(f & 63, nt - 1);  // past the block: its last token
        st.w[k] = *reinterpret_cast<const float4*>(wsc + ((int64_t)(tb + tt) * H + h) * ld + j0 + 4 * (f >> 6));
        const int j = min(j0 + (f >> 4), n_hi - 1);  // past n_hi: a re-read, never used
        st.v[k] = Cache<CT>::ldr(vbase + (int64_t)j * row + min(4 * (f & 15), ncol - 4));
    }
}

template <typename CT>
__device__ __forceinline__ void mt_pv_store(const MtPvStage<CT>& st, float* Wt, float* Vs) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int f = (int)threadIdx.x + kPvThreads2 * k, tt = f & 63, r = 4 * (f >> 6);
        Wt[(r + 0) * kPvTok + tt] = st.w[k].x;
        Wt[(r + 1) * kPvTok + tt] = st.w[k].y;
        Wt[(r + 2) * kPvTok + tt] = st.w[k].z;
        Wt[(r + 3) * kPvTok + tt] = st.w[k].w;
        reinterpret_cast<float4*>(Vs)[f] = Cache<CT>::cvt(st.v[k]);
    }
}

__device__ __forceinline__ void pv_fma42(float (&acc)[4][2], const float2& v, const float4& w) {
    const float wk[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        acc[k][0] = acc[k][0] + v.x * wk[k];
        acc[k][1] = acc[k][1] + v.y * wk[k];
    }
}

// Token block tb .. tb + nt - 1 of head h, columns d0 .. d0 + 63, by all 8 waves.
template <typename CT>
__device__ __forceinline__ void mt_pv_block(float (*Wt)[kScoreRows * kPvTok], float (*Vs)[kScoreRows * kPvCols],
                                            const float* __restrict__ wsc, const CT* __restrict__ vc,
                                            float* __restrict__ out, uint8_t* __restrict__ xq, int ld, int kv_pos,
                                            int tb, int nt, int h, int H, int HKV, int D, int d0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, th = wave >> 1, ch = wave & 1;
    const int tg = lane >> 4, cg = lane & 15;
    const int n_hi = kv_pos + tb + nt, nch = (n_hi + kScoreRows - 1) / kScoreRows;
    const int kvh = h / (H / HKV), row = HKV * D, ncol = min(kPvCols, D - d0);
    const CT* vbase = vc + (int64_t)kvh * D + d0;
    const int tw = 16 * th + 4 * tg, cw = 32 * ch + 2 * cg;  // the lane's first token and column in the block
    // rows of the wave's first token, and of the lane's 4 tokens
    const int n_wave = kv_pos + tb + 16 * th + 1, n_lane = kv_pos + tb + tw + 1;
    float acc[4][2];
#pragma unroll
    for (int k = 0; k < 4; k++) acc[k][0] = acc[k][1] = 0.0f;
    MtPvStage<CT> st;
    mt_pv_load<CT>(st, wsc, vbase, 0, tb, nt, h, H, ld, n_hi, row, ncol);
    mt_pv_store<CT>(st, Wt[0], Vs[0]);
    if (nch > 1) mt_pv_load<CT>(st, wsc, vbase, kScoreRows, tb, nt, h, H, ld, n_hi, row, ncol);
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        const int j0 = c * kScoreRows;
        const float2* v2 = reinterpret_cast<const float2*>(Vs[c & 1] + cw);
        const float4* w4 = reinterpret_cast<const float4*>(Wt[c & 1] + tw);
        if (j0 + kScoreRows <= n_wave) {  // every token of the wave has all 64 rows (uniform)
#pragma unroll 4
            for (int jj = 0; jj < kScoreRows; jj++) pv_fma42(acc, v2[jj * (kPvCols / 2)], w4[jj * (kPvTok / 4)]);
        } else if (j0 < n_wave + 15) {  // some token of the wave has rows here
            for (int jj = 0; jj < kScoreRows; jj++) {
                const float2 v = v2[jj * (kPvCols / 2)];
                const float4 w = w4[jj * (kPvTok / 4)];
                const float wk[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const bool on = j0 + jj < n_lane + k;  // row inside token tw + k's count
                    acc[k][0] = on ? acc[k][0] + v.x * wk[k] : acc[k][0];
                    acc[k][1] = on ? acc[k][1] + v.y * wk[k] : acc[k][1];
                }
            }
        }
        // the other slot was last read before the previous barrier
        if (c + 1 < nch) mt_pv_store<CT>(st, Wt[(c + 1) & 1], Vs[(c + 1) & 1]);
        if (c + 2 < nch) mt_pv_load<CT>(st, wsc, vbase, (c + 2) * kScoreRows, tb, nt, h, H, ld, n_hi, row, ncol);
        __syncthreads();
    }
    if (cw >= ncol) return;  // whole 16-lane groups (ncol is a multiple of 32)
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (tw + k >= nt) break;
        const int64_t o = ((int64_t)(tb + tw + k) * H + h) * D + d0 + cw;
        const float2 r = make_float2(acc[k][0], acc[k][1]);
        *reinterpret_cast<float2*>(out + o) = r;
        // Q8_0 of the token's 32 columns of this wave: the 16 lanes of tg, 2 each
        if (xq != nullptr) q8_0_pair_store(r, xq + (o >> 5) * kQ80Bytes, cg);
    }
}

template <typename CT>
__global__ __launch_bounds__(kPvThreads2) void k_mt_pv(const float* __restrict__ wsc, const CT* __restrict__ vc,
                                                        float* __restrict__ out, uint8_t* __restrict__ xq, int ld,
                                                        int kv_pos, int T, int H, int HKV, int D) {
    __shared__ __align__(16) float Wt[2][kScoreRows * kPvTok];   // [slot][row][token]
    __shared__ __align__(16) float Vs[2][kScoreRows * kPvCols];  // [slot][row][column]
    const int h = blockIdx.x, p = blockIdx.y, d0 = kPvCols * blockIdx.z, nb = (T + kPvTok - 1) / kPvTok;
    const int heavy = nb - 1 - p;
    mt_pv_block<CT>(Wt, Vs, wsc, vc, out, xq, ld, kv_pos, heavy * kPvTok, min(kPvTok, T - heavy * kPvTok), h, H, HKV, D,
                    d0);
    // the last barrier of the block above ends every read of both slots
    if (p != heavy) mt_pv_block<CT>(Wt, Vs, wsc, vc, out, xq, ld, kv_pos, p * kPvTok, kPvTok, h, H, HKV, D, d0);
}

// x = x + y over n floats (bpd_add_f32_cpu, bench/bpd_cpu.c:5466), n % 4 == 0.
__global__ __launch_bounds__(256) void k_add(float* __restrict__ x, const float* __restrict__ y, int64_t n4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float4 a = reinterpret_cast<float4*>(x)[i];
    const float4 b = reinterpret_cast<const float4*>(y)[i];
    a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    reinterpret_cast<float4*>(x)[i] = a;
}

// ---------------------------------------------------------------------------- host side

namespace {

template <typename CT>
hipError_t lds_limits_for() {
    hipError_t err = hipSuccess;
    for (const void* f : {reinterpret_cast<const void*>(&k_attn_pv<64, 32, CT>),
                          reinterpret_cast<const void*>(&k_attn_pv<64, 16, CT>)})
        if (err == hipSuccess) err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxCtx * 4);
    for (const void* f : {reinterpret_cast<const void*>(&k_attn_pv<128, 32, CT>),
                          reinterpret_cast<const void*>(&k_attn_pv<128, 16, CT>)})
        if (err == hipSuccess) err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPvBigMax * 4);
    // the scores kernels' LDS: the k tile plus q of up to n_embd / head_dim heads
    for (const void* f : {reinterpret_cast<const void*>(&k_attn_scores<128, CT>),
                          reinterpret_cast<const void*>(&k_attn_scores<64, CT>),
                          reinterpret_cast<const void*>(&k_attn_scores<0, CT>),
                          reinterpret_cast<const void*>(&k_mt_scores<CT>)})
        if (err == hipSuccess)
            err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (kScoreRows * score_pitch(kMaxHeadDim) + kMaxEmbd + 2 * kMaxHeadDim + 4) * 4);
    for (const void* f : {reinterpret_cast<const void*>(&k_mt_scores_tile<CT, 16>),
                          reinterpret_cast<const void*>(&k_mt_scores_tile<CT, 8>),
                          reinterpret_cast<const void*>(&k_mt_scores_tile<CT, 4>),
                          reinterpret_cast<const void*>(&k_mt_scores_tile<CT, 2>)})
        if (err == hipSuccess) err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    return err;
}
static_assert(mt_sm_lds(kMtSmGroup) <= 160 * 1024, "k_mt_softmax LDS");
hipError_t lds_limits_softmax() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&k_mt_softmax<kMtSmThreads>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)mt_sm_lds(kMtSmGroup));
}

// The kernels that take more than 64 KB of dynamic LDS say so once per process.
bool lds_limits_set(const char* fn) {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = lds_limits_for<float>();
        if (err == hipSuccess) err = lds_limits_for<uint16_t>();
        if (err == hipSuccess) err = lds_limits_softmax();
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_residual_rmsnorm<kNormThreads, kNormChunks>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kMaxEmbd * 4);
    });
    return abi_hip_ok(err, fn);
}

void launch_norm(const float* x_in, const float* add, float* x_out, const float* w, float* h, uint8_t* xq, int n,
                 float eps, hipStream_t s, uint8_t* xk = nullptr, int rows = 1) {
    hipLaunchKernelGGL((k_residual_rmsnorm<kNormThreads, kNormChunks>), dim3(rows), dim3(kNormThreads), (size_t)n * 4,
                       s, x_in, add, x_out, w, h, xq, xk, n, eps);
}

// Rotation table for `pos`: pair j < n_dims/2 turns by pos * theta_scale^j /
// freqs[j] (freqs NULL: no factor), the angle accumulated in fp32 exactly as
// the reference's loop does (bpd_rope_norm_freqs_cpu, bench/bpd_cpu.c:5158-5171:
// theta_scale = powf(base, -2/n_dims); theta_eff = theta / ff; theta *=
// theta_scale after each pair).  sincosf through a pointer, so the compiler
// neither folds nor reorders it.
template <typename F>
void rope_angles(int pos, int n_dims, float base, const float* freqs, F&& put) {
    static void (*volatile sc)(float, float*, float*) = sincosf;
    static float (*volatile pw)(float, float) = powf;
    const float theta_scale = pw(base, -2.0f / (float)n_dims);
    float theta = (float)pos;
    for (int j = 0; j < n_dims / 2; j++) {
        const float ff = freqs != nullptr ? freqs[j] : 1.0f;
        const float theta_eff = theta / ff;
        float s, c;
        sc(theta_eff, &s, &c);
        put(j, c, s);
        theta *= theta_scale;
    }
}
void rope_table(RopeTab& t, int pos, int n_dims, float base, const float* freqs) {
    rope_angles(pos, n_dims, base, freqs, [&](int j, float c, float s) {
        t.c[j] = c;
        t.s[j] = s;
    });
}

struct V {
    const char* fn;
    bool ok = true;
    void fail(int code, const char* what) {
        if (ok) abi_error(code, fn, what);
        ok = false;
    }
    void need(bool cond, int code, const char* what) {
        if (!cond) fail(code, what);
    }
    void ptr(const void* p, uintptr_t align, const char* name) {
        if (!ok) return;
        char buf[128];
        if (p == nullptr) {
            std::snprintf(buf, sizeof buf, "%s is NULL", name);
            fail(BPDQ_ERR_NULL, buf);
        } else if ((reinterpret_cast<uintptr_t>(p) & (align - 1)) != 0) {
            std::snprintf(buf, sizeof buf, "%s is not %d-byte aligned", name, (int)align);
            fail(BPDQ_ERR_ALIGN, buf);
        }
    }
    void dims(int got_k, int want_k, int got_n, int want_n, int layer, const char* name) {
        if (!ok || (got_k == want_k && got_n == want_n)) return;
        char buf[160];
        std::snprintf(buf, sizeof buf, "layer %d %s is %d x %d (K x N), expected %d x %d", layer, name, got_k, got_n,
                      want_k, want_n);
        fail(BPDQ_ERR_SHAPE, buf);
    }
};

struct Geometry {
    int E, H, HKV, D, F, L;
};

// Options of the extended step (bpd_llama_step_ext_gpu); the plain entry
// points use one format everywhere, rope_dim = head_dim, no frequency factors
// and fp32 caches.
struct StepOpts {
    const int* layer_formats;  // host [n_layers][7] or NULL
    int base_format, lm_format;
    int rope_dim;
    const float* rope_freqs;
    bool f16;
    int fmt(int layer, int m) const { return layer_formats ? layer_formats[layer * 7 + m] : base_format; }
};

bool is_q4k(int f) { return f == BPDQ_W_Q4K || f == BPDQ_W_Q4K_GGUF; }
bool is_q6k(int f) { return f == BPDQ_W_Q6K || f == BPDQ_W_Q6K_GGUF; }
bool known_format(int f) { return f == BPDQ_W_Q8_PAD64 || is_q4k(f) || is_q6k(f); }
int format_order(int f) { return f == BPDQ_W_Q4K_GGUF || f == BPDQ_W_Q6K_GGUF ? 1 : 0; }
uintptr_t format_align(int f) { return f == BPDQ_W_Q8_PAD64 ? 4 : is_q6k(f) ? 2 : 16; }

bool validate(V& v, const StepOpts& o, const LayerWeights* layers, const ModelConfig* cfg, const WorkBuffers* buf,
              const KVCache* kv, int pos, const void* emb, const void* out_norm, const void* lm_w,
              const void* lm_f32, int lm_K, int lm_N, Geometry& g) {
    v.ptr(cfg, 1, "cfg");
    v.ptr(buf, 1, "buf");
    if (!v.ok) return false;
    g = Geometry{cfg->n_embd, cfg->n_head, cfg->n_head_kv, cfg->head_dim, cfg->ff_dim, cfg->n_layers};
    v.need(g.L >= 0, BPDQ_ERR_SHAPE, "n_layers is negative");
    if (!v.ok) return false;
    // every matrix in padded Q8 (Q8_0 activations), or every one a K-quant (Q8_K activations)
    const bool q8 = o.base_format == BPDQ_W_Q8_PAD64;
    v.need(known_format(o.base_format), BPDQ_ERR_SHAPE, "unknown weight_format");
    for (int l = 0; l < g.L && v.ok; l++)
        for (int m = 0; m < 7 && v.ok; m++) {
            const int f = o.fmt(l, m);
            v.need(known_format(f), BPDQ_ERR_SHAPE, "unknown format in layer_formats");
            v.need((f == BPDQ_W_Q8_PAD64) == q8, BPDQ_ERR_SHAPE,
                   "the padded Q8 layout cannot be mixed with the K-quant formats");
        }
    if (lm_w != nullptr) {
        v.need(known_format(o.lm_format), BPDQ_ERR_SHAPE, "unknown lm_format");
        v.need((o.lm_format == BPDQ_W_Q8_PAD64) == q8, BPDQ_ERR_SHAPE,
               "the padded Q8 layout cannot be mixed with the K-quant formats");
    }
    if (!v.ok) return false;
    const int blk = q8 ? 32 : 256;
    v.need(g.H > 0 && g.HKV > 0 && g.H % g.HKV == 0, BPDQ_ERR_SHAPE,
           "n_head and n_head_kv must be positive, n_head a multiple of n_head_kv");
    v.need(g.D > 0 && g.D % 32 == 0 && g.D <= kMaxHeadDim, BPDQ_ERR_SHAPE,
           "head_dim must be a multiple of 32 and at most 256");
    v.need(g.E == g.H * g.D, BPDQ_ERR_SHAPE, "n_embd must equal n_head * head_dim");
    v.need(g.E > 0 && g.E % blk == 0 && g.E <= kMaxEmbd, BPDQ_ERR_SHAPE,
           "n_embd must be a positive multiple of the weight block length, at most 16384");
    v.need(g.F > 0 && g.F % blk == 0, BPDQ_ERR_SHAPE, "ff_dim must be a positive multiple of the weight block length");
    v.need(cfg->max_seq > 0 && cfg->max_seq <= kMaxCtx, BPDQ_ERR_SHAPE, "max_seq must be in 1..32768");
    v.need(pos >= 0 && pos < cfg->max_seq, BPDQ_ERR_SHAPE, "position must be in 0..max_seq-1");
    v.need(o.rope_dim >= 2 && o.rope_dim <= g.D && o.rope_dim % 2 == 0, BPDQ_ERR_SHAPE,
           "rope_dim must be even, in 2..head_dim");
    v.need(lm_K == g.E, BPDQ_ERR_SHAPE, "lm_K must equal n_embd");
    v.need(lm_N > 0, BPDQ_ERR_SHAPE, "lm_N must be positive");
    if (!v.ok) return false;
    v.ptr(emb, 16, "embedding");
    v.ptr(out_norm, 16, "output_norm_w");
    if (lm_w != nullptr)
        v.ptr(lm_w, format_align(o.lm_format), "lm_head");
    else
        v.ptr(lm_f32, 4, "lm_f32 (lm_head is NULL)");
    const void* bufs[11] = {buf->x, buf->h, buf->q, buf->k, buf->v, buf->attn_out,
                            buf->gate, buf->up, buf->ffn, buf->logits, buf->argmax_result};
    static const char* names[11] = {"buf.x", "buf.h", "buf.q", "buf.k", "buf.v", "buf.attn_out",
                                    "buf.gate", "buf.up", "buf.ffn", "buf.logits", "buf.argmax_result"};
    for (int i = 0; i < 11; i++) v.ptr(bufs[i], 16, names[i]);
    if (g.L > 0) {
        v.ptr(layers, 1, "layers");
        v.ptr(kv, 1, "kv");
        if (v.ok) {
            v.ptr(kv->k_cache, 1, "kv.k_cache");
            v.ptr(kv->v_cache, 1, "kv.v_cache");
        }
    }
    for (int l = 0; l < g.L && v.ok; l++) {
        const LayerWeights& w = layers[l];
        const int qd = g.H * g.D, kd = g.HKV * g.D;
        v.dims(w.q_K, g.E, w.q_N, qd, l, "q");
        v.dims(w.k_K, g.E, w.k_N, kd, l, "k");
        v.dims(w.v_K, g.E, w.v_N, kd, l, "v");
        v.dims(w.o_K, qd, w.o_N, g.E, l, "o");
        v.dims(w.gate_K, g.E, w.gate_N, g.F, l, "gate");
        v.dims(w.up_K, g.E, w.up_N, g.F, l, "up");
        v.dims(w.down_K, g.F, w.down_N, g.E, l, "down");
        const void* mats[7] = {w.q, w.k, w.v, w.o, w.gate, w.up, w.down};
        static const char* mnames[7] = {"q", "k", "v", "o", "gate", "up", "down"};
        for (int i = 0; i < 7; i++) v.ptr(mats[i], format_align(o.fmt(l, i)), mnames[i]);
        v.ptr(w.attn_norm, 16, "attn_norm");
        v.ptr(w.ffn_norm, 16, "ffn_norm");
        if (w.q_bias) v.ptr(w.q_bias, 4, "q_bias");
        if (w.k_bias) v.ptr(w.k_bias, 4, "k_bias");
        if (w.v_bias) v.ptr(w.v_bias, 4, "v_bias");
        v.ptr(kv->k_cache[l], 16, "kv.k_cache[layer]");
        v.ptr(kv->v_cache[l], 16, "kv.v_cache[layer]");
    }
    return v.ok;
}

// The GEMVs y_i[N_i] = W_i[N_i][K] a[K] of matrices that share one activation.
// Padded Q8 reads the Q8_0 bytes aq of a.  The K-quants read a's Q8_K: xk when
// the norm wrote it, else Q4_K quantizes inside the kernel (K <= fused_max_k())
// and Q6_K (or a longer Q4_K) reads q8k, written here once per group.  Q4_K
// matrices of one element map share a launch.
struct Gemv {
    uint8_t* q8k;  // Q8_K staging (K-quant formats)
    hipStream_t s;
    void run(int n, const void* const* w, const int* fmt, float* const* y, const int* N, const float* a,
             const uint8_t* aq, const uint8_t* xk, int K) const {
        if (fmt[0] == BPDQ_W_Q8_PAD64) {
            for (int i = 0; i < n; i++)
                launch_q8_pad64_dispatch_T(static_cast<const uint8_t*>(w[i]), aq, y[i], N[i], 1, K, s);
            return;
        }
        bool need_q8k = false;
        for (int i = 0; i < n; i++) need_q8k |= is_q6k(fmt[i]) || (is_q4k(fmt[i]) && K > fused_max_k());
        if (xk == nullptr && need_q8k) {
            launch_quant_q8k(a, q8k, K, s);
            xk = q8k;
        }
        for (int order = 0; order < 2; order++) {
            const uint8_t* wl[4];
            float* yl[4];
            int nl[4], m = 0;
            for (int i = 0; i < n; i++)
                if (is_q4k(fmt[i]) && format_order(fmt[i]) == order) {
                    wl[m] = static_cast<const uint8_t*>(w[i]);
                    yl[m] = y[i];
                    nl[m++] = N[i];
                }
            if (m == 0) continue;
            if (xk != nullptr)
                launch_qmatmul_q4k_q8k_multi(wl, yl, nl, m, xk, K, order, s);
            else
                launch_qmatmul_q4k_fused_multi(wl, yl, nl, m, a, K, order, s);
        }
        for (int i = 0; i < n; i++)
            if (is_q6k(fmt[i]))
                launch_qmatmul_q6k_q8k(static_cast<const uint8_t*>(w[i]), xk, y[i], N[i], K, format_order(fmt[i]), s);
    }
};

struct StepCtx {
    Geometry g;
    const ModelConfig* cfg;
    const KVCache* kv;
    const StepOpts* o;
    int pos;
    hipStream_t s;
    RopeTab tab;
    float *x, *h, *qb, *kb, *vb, *att, *gate, *up, *ffn;
    float* scores;      // [n_head][max_seq] scaled scores of the long-context attention
    float attn_scale;   // 1 / sqrtf(head_dim), as the reference computes it
    uint8_t *xq_e, *xq_a, *xq_f;  // Q8_0 activations (padded Q8 weights only, else NULL)
    uint8_t* xk;  // Q8_K of the normed row (K-quant weights, n_embd <= 4096, else NULL)
    double *part_o, *part_d;  // partial sums of squares of the O and down epilogues (norm folding)
    bool fold;                // RMSNorms folded into the GEMVs (see fold_norms)
};

// Whether every layer's norms can fold into its GEMVs (launch_q4k_res /
// launch_q4k_norm_*): n_embd 4096, ff_dim 4096 or 14336, all seven matrices Q4_K
// of one element map, 16-byte aligned, n_head * head_dim = n_embd.  Measured at cfg3: the two norm launches
// took 9.1 us of a 46 us layer at position 0.
bool fold_norms(const StepOpts& o, const Geometry& g, const LayerWeights* layers) {
    if (!norm_fusion_fits(g.E, g.F) || g.H * g.D != g.E || !is_q4k(o.base_format)) return false;
    for (int l = 0; l < g.L; l++) {
        const void* m[7] = {layers[l].q, layers[l].k, layers[l].v, layers[l].o, layers[l].gate, layers[l].up,
                            layers[l].down};
        for (int i = 0; i < 7; i++)
            if (o.fmt(l, i) != o.base_format || (reinterpret_cast<uintptr_t>(m[i]) & 15) != 0) return false;
    }
    return true;
}

// Attention over n_ctx = pos + 1 rows: one kernel while the context is short
// and head_dim is 32, 64 or 128, else scores and softmax/P.V as two kernels.
template <typename CT>
void attention(const StepCtx& c, const AttnIn& ai, int n_ctx) {
    const Geometry& g = c.g;
    if (n_ctx <= kSmallCtx && (g.D == 32 || g.D == 64 || g.D == 128)) {
        if (g.D == 128)
            hipLaunchKernelGGL((k_attn_small<128, CT>), dim3(g.H), dim3(256), 0, c.s, ai, c.tab, c.att, c.xq_a);
        else if (g.D == 64)
            hipLaunchKernelGGL((k_attn_small<64, CT>), dim3(g.H), dim3(256), 0, c.s, ai, c.tab, c.att, c.xq_a);
        else
            hipLaunchKernelGGL((k_attn_small<32, CT>), dim3(g.H), dim3(256), 0, c.s, ai, c.tab, c.att, c.xq_a);
        return;
    }
    const int ld = c.cfg->max_seq, group = g.H / g.HKV;
    const dim3 gs(g.HKV * ((n_ctx + kScoreRows - 1) / kScoreRows)), ts(64 * (group < kMaxGroup ? group : kMaxGroup));
    // k tile, q of the group's heads, new k and v rows, a spare float4: <= (64 * 260 + 16384 + 516) * 4 bytes
    const size_t slds = ((size_t)kScoreRows * score_pitch(g.D) + (size_t)(group + 2) * g.D + 4) * 4;
    if (g.D == 128)
        hipLaunchKernelGGL((k_attn_scores<128, CT>), gs, ts, slds, c.s, ai, c.tab, c.scores, ld);
    else if (g.D == 64)
        hipLaunchKernelGGL((k_attn_scores<64, CT>), gs, ts, slds, c.s, ai, c.tab, c.scores, ld);
    else
        hipLaunchKernelGGL((k_attn_scores<0, CT>), gs, ts, slds, c.s, ai, c.tab, c.scores, ld);
    // e holds pad64(n_ctx) <= kMaxCtx floats (kMaxCtx % 64 == 0); with 128-row
    // chunks n_ctx <= kPvBigMax, so the ring and the scores fit in 160 KB
    // 16-column slices unless the output's Q8_0 bytes are wanted (head_dim % 32 == 0)
    const size_t lds = (size_t)pad64(n_ctx) * 4;
    const bool big = n_ctx >= kPvBigMin && n_ctx <= kPvBigMax;
    if (c.xq_a == nullptr) {
        const dim3 gp(g.H * (g.D / 16));
        if (big)
            hipLaunchKernelGGL((k_attn_pv<128, 16, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, ld, c.att, nullptr);
        else
            hipLaunchKernelGGL((k_attn_pv<64, 16, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, ld, c.att, nullptr);
    } else {
        const dim3 gp(g.H * (g.D / 32));
        if (big)
            hipLaunchKernelGGL((k_attn_pv<128, 32, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, ld, c.att, c.xq_a);
        else
            hipLaunchKernelGGL((k_attn_pv<64, 32, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, ld, c.att, c.xq_a);
    }
}

// The layers.  The residual add is the first step of each RMSNorm kernel; the
// norm, attention and SwiGLU kernels also write the Q8_0 bytes of their outputs
// when the GEMVs take Q8_0 activations.  On return (xin, add) is the residual
// stream as x + add.
void run_layers(const StepCtx& c, const Gemv& gemv, const LayerWeights* layers, const float*& xin,
                const float*& add) {
    const Geometry& g = c.g;
    const StepOpts& o = *c.o;
    const int row = g.HKV * g.D, n_ctx = c.pos + 1;
    int npart_d = 0;  // partials of the previous layer's down epilogue
    for (int l = 0; l < g.L; l++) {
        const LayerWeights& w = layers[l];
        int f[7];
        for (int m = 0; m < 7; m++) f[m] = o.fmt(l, m);
        const void* wqkv[3] = {w.q, w.k, w.v};
        float* yqkv[3] = {c.qb, c.kb, c.vb};
        const int nqkv[3] = {w.q_N, w.k_N, w.v_N};
        if (c.fold && l > 0) {  // the norm from the residual row and the down epilogue's partials
            const uint8_t* wl[3] = {static_cast<const uint8_t*>(w.q), static_cast<const uint8_t*>(w.k),
                                    static_cast<const uint8_t*>(w.v)};
            const NormIn nin{c.x, static_cast<const float*>(w.attn_norm), c.part_d, npart_d, c.cfg->eps};
            launch_q4k_norm_multi(wl, yqkv, nqkv, 3, nin, format_order(f[0]), c.s);
        } else {
            launch_norm(xin, add, c.x, static_cast<const float*>(w.attn_norm), c.h, c.xq_e, g.E, c.cfg->eps, c.s,
                        c.xk);
            gemv.run(3, wqkv, f, yqkv, nqkv, c.h, c.xq_e, c.xk, g.E);
        }
        xin = c.x;
        const AttnIn ai{c.qb, c.kb, c.vb,
                        static_cast<const float*>(w.q_bias), static_cast<const float*>(w.k_bias),
                        static_cast<const float*>(w.v_bias), c.kv->k_cache[l], c.kv->v_cache[l], g.H / g.HKV, row,
                        g.D, c.pos, c.attn_scale, o.rope_dim / 2};
        if (o.f16)
            attention<uint16_t>(c, ai, n_ctx);
        else
            attention<float>(c, ai, n_ctx);
        if (c.fold) {  // O into the residual row, gate/up with the norm, down into the residual row
            const int ord = format_order(f[0]);
            const int npart_o = launch_q4k_res(static_cast<const uint8_t*>(w.o), w.o_N, c.att, g.H * g.D,
                                               ResOut{c.x, c.part_o}, ord, c.s);
            const NormIn nin{c.x, static_cast<const float*>(w.ffn_norm), c.part_o, npart_o, c.cfg->eps};
            hipLaunchKernelGGL(k_norm_q8k, dim3(g.E / 256), dim3(64), 0, c.s, nin, c.xk);
            launch_qmatmul_q4k_swiglu_q8k(static_cast<const uint8_t*>(w.gate), static_cast<const uint8_t*>(w.up),
                                          c.gate, g.F, c.xk, g.E, ord, c.s);
            npart_d = launch_q4k_res(static_cast<const uint8_t*>(w.down), w.down_N, c.gate, g.F, ResOut{c.x, c.part_d},
                                     ord, c.s);
            add = nullptr;
            continue;
        }
        const void* wo[1] = {w.o};
        float* yo[1] = {c.ffn};
        const int no[1] = {w.o_N};
        gemv.run(1, wo, f + 3, yo, no, c.att, c.xq_a, nullptr, g.H * g.D);
        launch_norm(c.x, c.ffn, c.x, static_cast<const float*>(w.ffn_norm), c.h, c.xq_e, g.E, c.cfg->eps, c.s, c.xk);
        // gate/up with SwiGLU in the epilogue (into gate) when both are Q4_K of one map
        const bool fused = is_q4k(f[4]) && f[4] == f[5];
        if (fused && c.xk != nullptr) {
            launch_qmatmul_q4k_swiglu_q8k(static_cast<const uint8_t*>(w.gate), static_cast<const uint8_t*>(w.up),
                                          c.gate, g.F, c.xk, g.E, format_order(f[4]), c.s);
        } else if (fused && g.E <= fused_max_k()) {
            launch_qmatmul_q4k_fused_swiglu(static_cast<const uint8_t*>(w.gate), static_cast<const uint8_t*>(w.up),
                                            c.gate, g.F, c.h, g.E, format_order(f[4]), c.s);
        } else {
            const void* wgu[2] = {w.gate, w.up};
            float* ygu[2] = {c.gate, c.up};
            const int ngu[2] = {w.gate_N, w.up_N};
            gemv.run(2, wgu, f + 4, ygu, ngu, c.h, c.xq_e, c.xk, g.E);
            hipLaunchKernelGGL(k_swiglu, dim3((g.F + 255) / 256), dim3(256), 0, c.s, c.gate, c.up, c.xq_f, g.F);
        }
        const void* wd[1] = {w.down};
        float* yd[1] = {c.ffn};
        const int nd[1] = {w.down_N};
        gemv.run(1, wd, f + 6, yd, nd, c.gate, c.xq_f, nullptr, g.F);
        add = c.ffn;
    }
}

bool enqueue_step(const StepOpts& o, const LayerWeights* layers, const ModelConfig* cfg, const WorkBuffers* buf,
                  const KVCache* kv, int pos, const void* emb, const void* out_norm, const void* lm_w,
                  const void* lm_f32, int lm_K, int lm_N, const char* fn) {
    V v{fn};
    StepCtx c{};
    Geometry& g = c.g;
    if (!validate(v, o, layers, cfg, buf, kv, pos, emb, out_norm, lm_w, lm_f32, lm_K, lm_N, g)) return false;
    if (!lds_limits_set(fn)) return false;
    const bool q8 = o.base_format == BPDQ_W_Q8_PAD64;
    const size_t q8e = (size_t)(g.E / 32) * kQ80Bytes, q8f = (size_t)(g.F / 32) * kQ80Bytes;
    const size_t front = q8 ? (2 * q8e + q8f + 255) & ~(size_t)255 : 0;
    const int kmax = g.F > g.E ? g.F : g.E;
    const size_t q8k = q8 ? 0 : (size_t)(kmax / 256) * kQ8KBytes;
    // with K-quant weights and n_embd <= 4096 the norms write h's Q8_K once for the
    // Q/K/V and gate/up GEMVs (measured 1,515 -> 1,500 us/token at cfg3)
    const size_t xk_bytes = !q8 && g.E <= 4096 ? ((size_t)(g.E / 256) * kQ8KBytes + 255) & ~(size_t)255 : 0;
    const size_t q8k_end = ((front + q8k + 255) & ~(size_t)255) + xk_bytes;
    const size_t sc_bytes = ((size_t)g.H * cfg->max_seq * 4 + 255) & ~(size_t)255;
    // two sets of per-workgroup partials (a producer workgroup has at least 4
    // waves of at least one row of n_embd)
    c.fold = xk_bytes != 0 && fold_norms(o, g, layers);
    const size_t part_bytes = c.fold ? 2 * ((((size_t)g.E / 4 + 1) * 8 + 255) & ~(size_t)255) : 0;
    // the quantized activations (Q8_0 rows, or Q8_K staging for the K-quant GEMVs),
    // the attention scores and the partials, in the stream's workspace
    const WsLease lease = workspace(q8k_end + sc_bytes + part_bytes, abi_stream(), fn);
    uint8_t* ws = static_cast<uint8_t*>(lease.ptr);
    if (ws == nullptr) return false;
    const Gemv gemv{ws + front, abi_stream()};
    c.cfg = cfg;
    c.kv = kv;
    c.o = &o;
    c.pos = pos;
    c.scores = reinterpret_cast<float*>(ws + q8k_end);
    c.attn_scale = 1.0f / sqrtf((float)g.D);
    c.s = gemv.s;
    c.x = static_cast<float*>(buf->x);
    c.h = static_cast<float*>(buf->h);
    c.qb = static_cast<float*>(buf->q);
    c.kb = static_cast<float*>(buf->k);
    c.vb = static_cast<float*>(buf->v);
    c.att = static_cast<float*>(buf->attn_out);
    c.gate = static_cast<float*>(buf->gate);
    c.up = static_cast<float*>(buf->up);
    c.ffn = static_cast<float*>(buf->ffn);
    c.xq_e = q8 ? ws : nullptr;
    c.xq_a = q8 ? ws + q8e : nullptr;
    c.xq_f = q8 ? ws + 2 * q8e : nullptr;
    c.xk = xk_bytes ? ws + q8k_end - xk_bytes : nullptr;
    if (c.fold) {
        c.part_o = reinterpret_cast<double*>(ws + q8k_end + sc_bytes);
        c.part_d = reinterpret_cast<double*>(ws + q8k_end + sc_bytes + part_bytes / 2);
    }
    if (g.L > 0) rope_table(c.tab, pos, o.rope_dim, cfg->rope_theta, o.rope_freqs);
    float* logits = static_cast<float*>(buf->logits);

    const float* xin = static_cast<const float*>(emb);
    const float* add = nullptr;
    run_layers(c, gemv, layers, xin, add);
    launch_norm(xin, add, c.x, static_cast<const float*>(out_norm), c.h, c.xq_e, g.E, cfg->eps, c.s, c.xk);
    if (lm_w != nullptr) {
        const void* wl[1] = {lm_w};
        const int fl[1] = {o.lm_format};
        float* yl[1] = {logits};
        const int nl[1] = {lm_N};
        gemv.run(1, wl, fl, yl, nl, c.h, c.xq_e, c.xk, g.E);
    } else {
        hipLaunchKernelGGL(k_gemv_f32, dim3((lm_N + 3) / 4), dim3(256), 0, c.s, static_cast<const float*>(lm_f32),
                           c.h, logits, lm_N, g.E);
    }
    hipLaunchKernelGGL(k_argmax<1024>, dim3(1), dim3(1024), 0, c.s, logits, lm_N,
                       static_cast<int32_t*>(buf->argmax_result), nullptr);
    return abi_hip_ok(hipGetLastError(), fn);
}

StepOpts plain_opts(int fmt, const ModelConfig* cfg) {
    return StepOpts{nullptr, fmt, fmt, cfg != nullptr ? cfg->head_dim : 0, nullptr, false};
}


// ---------------------------------------------------------------------------- several tokens
// bpd_llama_block_cpu / bpd_llama_forward_cpu (bench/bpd_cpu.c:5608-5798) for
// n_tokens >= 1.  Per layer, as the reference's block: RMSNorm of every row;
// Q, K, V; RoPE of q and k and the cache writes of every token; attention of
// query t over cache rows 0..kv_pos+t; O; x += O; RMSNorm; gate, up; SwiGLU;
// down; x += down.  The Q8_0 products are the llamafile entry's (quantize the
// rows, then the tile order T of the -mavx build, or order S of the -O2 build
// on int8 MFMA); every other operation is shared by both builds.

struct BlockGeo {
    int E, H, HKV, D, F, S, rot;
    bool f16;
    float eps, base;
};

bool validate_block_cfg(V& v, const bpd_llama_config* cfg, int T, int kv_pos, const int32_t* pos_ids, BlockGeo& g) {
    v.ptr(cfg, 1, "cfg");
    if (!v.ok) return false;
    g = BlockGeo{cfg->embed_dim, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, cfg->ffn_dim, cfg->max_seq_len,
                 cfg->rope_dim / 2, cfg->kv_cache_f16 != 0, cfg->rms_eps, cfg->rope_base};
    v.need(T >= 0, BPDQ_ERR_SHAPE, "n_tokens is negative");
    v.need(g.H > 0 && g.HKV > 0 && g.H % g.HKV == 0, BPDQ_ERR_SHAPE,
           "n_heads and n_kv_heads must be positive, n_heads a multiple of n_kv_heads");
    v.need(g.D > 0 && g.D % 32 == 0 && g.D <= kMaxHeadDim, BPDQ_ERR_SHAPE,
           "head_dim must be a multiple of 32 and at most 256");
    v.need(g.E == g.H * g.D && g.E <= kMaxEmbd, BPDQ_ERR_SHAPE, "embed_dim must equal n_heads * head_dim, at most 16384");
    v.need(g.F > 0 && g.F % 32 == 0, BPDQ_ERR_SHAPE, "ffn_dim must be a positive multiple of 32");
    v.need(cfg->rope_dim >= 2 && cfg->rope_dim <= g.D && cfg->rope_dim % 2 == 0, BPDQ_ERR_SHAPE,
           "rope_dim must be even, in 2..head_dim");
    v.need(g.S > 0 && g.S <= kMaxCtx, BPDQ_ERR_SHAPE, "max_seq_len must be in 1..32768");
    v.need(kv_pos >= 0 && (int64_t)kv_pos + T <= g.S, BPDQ_ERR_SHAPE, "kv_pos + n_tokens must be in 0..max_seq_len");
    if (!v.ok || T == 0) return v.ok;
    v.ptr(pos_ids, 4, "pos_ids");
    for (int t = 0; t < T && v.ok; t++)
        v.need(pos_ids[t] >= 0 && pos_ids[t] < g.S, BPDQ_ERR_SHAPE, "pos_ids[t] must be in 0..max_seq_len-1");
    return v.ok;
}

void validate_layer(V& v, const bpd_llama_layer_weights* lw, const void* kc, const void* vc) {
    v.ptr(lw, 1, "layer weights");
    if (!v.ok) return;
    v.ptr(lw->attn_norm_w, 16, "attn_norm_w");
    v.ptr(lw->ffn_norm_w, 16, "ffn_norm_w");
    const void* m[7] = {lw->w_q, lw->w_k, lw->w_v, lw->w_o, lw->w_gate, lw->w_up, lw->w_down};
    static const char* names[7] = {"w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down"};
    for (int i = 0; i < 7; i++) v.ptr(m[i], 1, names[i]);
    v.ptr(kc, 16, "k_cache");
    v.ptr(vc, 16, "v_cache");
}

constexpr int kRopeSlots = kMaxHeadDim / 2;  // RopeCS entries per token

struct MtCtx {
    BlockGeo g;
    int T, kv_pos;
    bool order_s;
    hipStream_t s;
    const int32_t* ids;   // device copies of the host arrays
    const int32_t* pos;
    const RopeCS* tab;    // [T][kRopeSlots]
    uint8_t* xq;          // Q8_0 rows of the current GEMM input, [T][max(E,F)/32][34]
    float* scores;        // [tc][H][ld]
    uint8_t* yq;          // Q8_0 rows of SwiGLU's y when gate/up write them, [T][F/32][34]
    int ld, tc;           // score row pitch (kv_pos + T rounded up to 64) and tokens per attention launch
    float scale;
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
size_t host_region_bytes(int T) { return 2 * align256((size_t)T * 4) + align256((size_t)T * kRopeSlots * sizeof(RopeCS)); }

// Workspace: [token ids | positions | rotation table] [Q8_0 rows] [scores] [extra]
// (extra: the forward's x and three scratch rows).  Fills c's pointers.
uint8_t* mt_workspace(MtCtx& c, WsLease& lease, size_t extra, const char* fn) {
    const BlockGeo& g = c.g;
    const int kmax = g.F > g.E ? g.F : g.E;
    c.ld = pad64(c.kv_pos + c.T);
    const size_t per_tok = (size_t)g.H * c.ld * 4;
    const size_t budget = (size_t)64 << 20;  // scores of at most 64 MiB per attention launch
    c.tc = (int)std::max<size_t>(1, std::min<size_t>(std::min<size_t>((size_t)c.T, 32768), budget / per_tok));
    const size_t hb = host_region_bytes(c.T), qb = align256((size_t)c.T * (kmax / 32) * kQ80Bytes);
    const size_t sb = align256((size_t)c.tc * per_tok), ib = align256((size_t)c.T * (g.F / 32) * kQ80Bytes);
    lease = workspace(hb + qb + sb + ib + extra, c.s, fn);
    uint8_t* ws = static_cast<uint8_t*>(lease.ptr);
    if (ws == nullptr) return nullptr;
    c.ids = reinterpret_cast<const int32_t*>(ws);
    c.pos = reinterpret_cast<const int32_t*>(ws + align256((size_t)c.T * 4));
    c.tab = reinterpret_cast<const RopeCS*>(ws + 2 * align256((size_t)c.T * 4));
    c.xq = ws + hb;
    c.scores = reinterpret_cast<float*>(ws + hb + qb);
    c.yq = ws + hb + qb + sb;
    return ws + hb + qb + sb + ib;
}

// Copies the token ids (or none), positions and rotation angles to the head of
// the workspace, then waits for the copy: the host arrays are the caller's.
bool mt_upload(const MtCtx& c, const int32_t* ids, const int32_t* pos_ids, const float* freqs, const char* fn) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!abi_hip_ok(hipStreamIsCapturing(c.s, &cs), fn)) return false;
    if (cs != hipStreamCaptureStatusNone) {
        abi_error(BPDQ_ERR_CAPTURE, fn, "the call uploads host arrays and waits for the copy: not under stream capture");
        return false;
    }
    const int T = c.T;
    std::vector<uint8_t> h(host_region_bytes(T), 0);
    if (ids != nullptr) std::memcpy(h.data(), ids, (size_t)T * 4);
    std::memcpy(h.data() + align256((size_t)T * 4), pos_ids, (size_t)T * 4);
    RopeCS* tab = reinterpret_cast<RopeCS*>(h.data() + 2 * align256((size_t)T * 4));
    for (int t = 0; t < T; t++)
        rope_angles(pos_ids[t], 2 * c.g.rot, c.g.base, freqs, [&](int j, float cv, float sv) {
            tab[(size_t)t * kRopeSlots + j] = RopeCS{cv, sv};
        });
    if (!abi_hip_ok(hipMemcpyAsync(const_cast<int32_t*>(c.ids), h.data(), h.size(), hipMemcpyHostToDevice, c.s), fn))
        return false;
    return abi_hip_ok(hipStreamSynchronize(c.s), fn);
}

// out[T][mw] = W[mw][K] . rows of xq (the Q8_0 rows of the input; c.xq by default).
void mt_gemm(const MtCtx& c, const uint8_t* W, float* out, int mw, int K, const uint8_t* xq = nullptr) {
    if (xq == nullptr) xq = c.xq;
    if (c.order_s)
        launch_q8_0_gemm_S(W, xq, out, mw, c.T, K, 1, c.s);  // the -O2 build's llamafile: qdot S per cell
    else
        launch_q8_0_dispatch_T(W, xq, out, mw, c.T, K, c.s);
}

// n GEMMs of the same activation rows (Q/K/V, gate/up): order S in one launch,
// order T one dispatch each.  (Q/K/V of 512 tokens of a Mistral-7B layer, 6144
// rows in all: 76 us in one launch against 174 us in three, each of which left
// most CUs idle.)
void mt_gemm3(const MtCtx& c, std::initializer_list<const uint8_t*> W, std::initializer_list<float*> out,
              std::initializer_list<int> M, int n, int K) {
    const uint8_t* w[3];
    float* o[3];
    int m[3];
    std::copy(W.begin(), W.end(), w);
    std::copy(out.begin(), out.end(), o);
    std::copy(M.begin(), M.end(), m);
    if (c.order_s) {
        launch_q8_0_gemm_S_multi(w, o, m, n, c.xq, c.T, K, 1, c.s);
        return;
    }
    for (int i = 0; i < n; i++) mt_gemm(c, w[i], o[i], m[i], K);
}

// Attention of the batch: out[T][H*D] and its Q8_0 rows in c.xq.  The tile
// kernels (k_mt_scores_tile, k_mt_softmax, k_mt_pv) when the scores tile fits in
// LDS (G * head_dim <= 2,048 at head_dim <= 256: every llama shape), otherwise
// the decode kernels with one grid row per token.
template <typename CT>
void mt_attention(const MtCtx& c, const float* q, const CT* kc, const CT* vc, float* out) {
    const BlockGeo& g = c.g;
    const int group = g.H / g.HKV;
    const int row = g.HKV * g.D;
    const bool tile = mt_scores_lds(group, g.D) <= 160 * 1024;
    const dim3 ts(64 * (group < kMaxGroup ? group : kMaxGroup));
    // the tile kernel's token subsets: as many as fit group heads each in 8 waves (1, 2, 4 or 8)
    const int reps = kMaxGroup / group >= 8 ? 8 : kMaxGroup / group >= 4 ? 4 : kMaxGroup / group >= 2 ? 2 : 1;
    const auto tile_k = reps == 8 ? &k_mt_scores_tile<CT, 2>
                        : reps == 4 ? &k_mt_scores_tile<CT, 4>
                        : reps == 2 ? &k_mt_scores_tile<CT, 8>
                                    : &k_mt_scores_tile<CT, 16>;
    for (int t0 = 0; t0 < c.T; t0 += c.tc) {
        const int tn = std::min(c.tc, c.T - t0), n_max = c.kv_pos + t0 + tn;
        float* o = out + (int64_t)t0 * g.H * g.D;
        uint8_t* xq = c.xq + (int64_t)t0 * (g.H * g.D / 32) * kQ80Bytes;
        const float* qt = q + (int64_t)t0 * g.H * g.D;
        if (tile) {
            const dim3 gs((n_max + kScoreRows - 1) / kScoreRows, g.HKV, (tn + kMtTok - 1) / kMtTok);
            hipLaunchKernelGGL(tile_k, gs, dim3(64 * kMaxGroup), mt_scores_lds(group, g.D), c.s, qt, kc, c.scores, c.ld,
                               c.kv_pos + t0, tn, g.H, g.HKV, g.D, c.scale);
            const int nb = (tn + kMtBlk - 1) / kMtBlk;
            hipLaunchKernelGGL((k_mt_softmax<kMtSmThreads>), dim3(g.H, nb), dim3(kMtSmThreads),
                               mt_sm_lds((n_max + kScoreRows - 1) / kScoreRows), c.s, c.scores, c.ld, c.kv_pos + t0,
                               tn, g.H);
            const int pairs = ((tn + kPvTok - 1) / kPvTok + 1) / 2;
            hipLaunchKernelGGL((k_mt_pv<CT>), dim3(g.H, pairs, (g.D + kPvCols - 1) / kPvCols), dim3(kPvThreads2), 0, c.s,
                               c.scores, vc, o, xq, c.ld, c.kv_pos + t0, tn, g.H, g.HKV, g.D);
            continue;
        }
        const size_t slds = ((size_t)kScoreRows * score_pitch(g.D) + (size_t)group * g.D + 4) * 4;
        const dim3 gs((n_max + kScoreRows - 1) / kScoreRows, g.HKV, tn);
        hipLaunchKernelGGL((k_mt_scores<CT>), gs, ts, slds, c.s, qt, kc, c.scores, c.ld, c.kv_pos + t0, g.H, g.HKV,
                           g.D, c.scale);
        const AttnIn ai{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, const_cast<CT*>(kc), const_cast<CT*>(vc),
                        group, row, g.D, c.kv_pos + t0, c.scale, c.g.rot};
        const dim3 gp(g.H * (g.D / 32), tn);
        const size_t lds = (size_t)pad64(n_max) * 4;
        if (n_max >= kPvBigMin && n_max <= kPvBigMax)
            hipLaunchKernelGGL((k_attn_pv<128, 32, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, c.ld, o, xq);
        else
            hipLaunchKernelGGL((k_attn_pv<64, 32, CT>), gp, dim3(kPvThreads), lds, c.s, ai, c.scores, c.ld, o, xq);
    }
}

// One layer over the batch x[T][E], with the reference block's use of its
// scratch rows: s1 = h, v, attention output, down output; s2 = q, O output,
// gate, SwiGLU; s3 = k, up; except that the norms write no h rows (their GEMMs
// read only the Q8_0 rows in c.xq) and order S with the SwiGLU epilogue writes
// no gate, up or SwiGLU rows (y goes to c.yq as Q8_0 only).
// add_in: the previous layer's down output, still to be added into x (the add
// then runs inside this layer's first norm: x = x + add_in, then its norm).
// defer_add: leave this layer's down output in s3 for the next norm instead of
// adding it into x here (s3 holds up, which SwiGLU has consumed by then).
template <typename CT>
void mt_layer(const MtCtx& c, float* x, const bpd_llama_layer_weights& w, CT* kc, CT* vc, float* s1, float* s2,
              float* s3, const float* add_in = nullptr, bool defer_add = false) {
    const BlockGeo& g = c.g;
    const int T = c.T, qd = g.H * g.D, kd = g.HKV * g.D;
    // the norms write only the Q8_0 rows their GEMM reads (no fp32 h rows)
    launch_norm(x, add_in, add_in != nullptr ? x : nullptr, w.attn_norm_w, nullptr, c.xq, g.E, g.eps, c.s, nullptr,
                T);
    mt_gemm3(c, {w.w_q, w.w_k, w.w_v}, {s2, s3, s1}, {qd, kd, kd}, 3, g.E);
    hipLaunchKernelGGL((k_rope_write<CT>), dim3(T), dim3(256), 0, c.s, s2, s3, s1, kc, vc, c.pos, c.tab, g.H, g.HKV,
                       g.D, g.rot);
    mt_attention<CT>(c, s2, kc, vc, s1);
    mt_gemm(c, w.w_o, s2, g.E, qd);
    launch_norm(x, s2, x, w.ffn_norm_w, nullptr, c.xq, g.E, g.eps, c.s, nullptr, T);
    // order S: SwiGLU and its Q8_0 rows in the gate/up GEMM's epilogue (into c.yq;
    // s2 and s3 then keep no gate, up or SwiGLU rows); otherwise k_swiglu
    const uint8_t* fq = nullptr;
    if (c.order_s && launch_q8_0_gemm_S_swiglu(w.w_gate, w.w_up, g.F, c.xq, T, g.E, 1, c.yq, c.s)) {
        fq = c.yq;
    } else {
        mt_gemm3(c, {w.w_gate, w.w_up, w.w_up}, {s2, s3, s3}, {g.F, g.F, g.F}, 2, g.E);
        const int64_t tf = (int64_t)T * g.F;
        hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((tf + 255) / 256)), dim3(256), 0, c.s, s2, s3, c.xq, (int)tf);
    }
    if (defer_add) {
        mt_gemm(c, w.w_down, s3, g.E, g.F, fq);
        return;
    }
    mt_gemm(c, w.w_down, s1, g.E, g.F, fq);
    const int64_t n4 = (int64_t)T * g.E / 4;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, c.s, x, s1, n4);
}

void llama_block(bool order_s, float* x, const bpd_llama_layer_weights* lw, const bpd_llama_config* cfg,
                 const int32_t* pos_ids, int T, int kv_pos, uint16_t* kc, uint16_t* vc, float* s1, float* s2,
                 float* s3, const float* freqs, const char* fn) {
    V v{fn};
    MtCtx c{};
    if (!validate_block_cfg(v, cfg, T, kv_pos, pos_ids, c.g) || T == 0) return;
    v.ptr(x, 16, "x");
    validate_layer(v, lw, kc, vc);
    v.ptr(s1, 16, "scratch1");
    v.ptr(s2, 16, "scratch2");
    v.ptr(s3, 16, "scratch3");
    if (!v.ok || !lds_limits_set(fn)) return;
    c.T = T;
    c.kv_pos = kv_pos;
    c.order_s = order_s;
    c.s = abi_stream();
    c.scale = 1.0f / sqrtf((float)c.g.D);
    WsLease lease;
    if (mt_workspace(c, lease, 0, fn) == nullptr) return;
    if (!mt_upload(c, nullptr, pos_ids, freqs, fn)) return;
    if (c.g.f16)
        mt_layer<uint16_t>(c, x, *lw, kc, vc, s1, s2, s3);
    else
        mt_layer<float>(c, x, *lw, reinterpret_cast<float*>(kc), reinterpret_cast<float*>(vc), s1, s2, s3);
    abi_hip_ok(hipGetLastError(), fn);
}

void llama_forward(bool order_s, const int32_t* ids, int T, const bpd_llama_weights* w, const bpd_llama_config* cfg,
                   const int32_t* pos_ids, int kv_pos, uint16_t* kc, uint16_t* vc, float* logits, int64_t* tok,
                   const char* fn) {
    V v{fn};
    MtCtx c{};
    if (!validate_block_cfg(v, cfg, T, kv_pos, pos_ids, c.g) || T == 0) return;
    const BlockGeo& g = c.g;
    v.ptr(w, 1, "weights");
    if (!v.ok) return;
    const int L = cfg->n_layers, NV = cfg->vocab_size;
    v.need(L >= 0, BPDQ_ERR_SHAPE, "n_layers is negative");
    v.need(NV > 0, BPDQ_ERR_SHAPE, "vocab_size must be positive");
    v.ptr(ids, 4, "token_ids");
    for (int t = 0; t < T && v.ok; t++) v.need(ids[t] >= 0 && ids[t] < NV, BPDQ_ERR_SHAPE, "token id outside 0..vocab_size-1");
    v.ptr(w->token_embd, 1, "token_embd");
    v.ptr(w->output_norm_w, 16, "output_norm_w");
    v.ptr(w->output_w, 1, "output_w");
    v.ptr(logits, 4, "logits_out");
    v.ptr(tok, 8, "token_out");
    if (L > 0) {
        v.ptr(w->layers, 1, "layers");
        v.ptr(kc, 16, "k_cache");
        v.ptr(vc, 16, "v_cache");
    }
    const size_t layer_elems = (size_t)g.S * g.HKV * g.D;
    const size_t esz = g.f16 ? 2 : 4;
    for (int l = 0; l < L && v.ok; l++)
        validate_layer(v, &w->layers[l], reinterpret_cast<uint8_t*>(kc) + l * layer_elems * esz,
                       reinterpret_cast<uint8_t*>(vc) + l * layer_elems * esz);
    if (!v.ok || !lds_limits_set(fn)) return;
    c.T = T;
    c.kv_pos = kv_pos;
    c.order_s = order_s;
    c.s = abi_stream();
    c.scale = 1.0f / sqrtf((float)g.D);
    const int kmax = g.F > g.E ? g.F : g.E;
    const size_t xb = align256((size_t)T * g.E * 4), sb = align256((size_t)T * kmax * 4);
    WsLease lease;
    uint8_t* extra = mt_workspace(c, lease, xb + 3 * sb, fn);
    if (extra == nullptr) return;
    if (!mt_upload(c, ids, pos_ids, w->rope_freqs, fn)) return;
    float* x = reinterpret_cast<float*>(extra);
    float* s1 = reinterpret_cast<float*>(extra + xb);
    float* s2 = reinterpret_cast<float*>(extra + xb + sb);
    float* s3 = reinterpret_cast<float*>(extra + xb + 2 * sb);
    launch_embed_q8_0(w->token_embd, c.ids, x, T, g.E, c.s);
    // each layer's residual add of its down output runs in the next norm (the
    // next layer's, or the final one)
    for (int l = 0; l < L; l++) {
        const float* add_in = l > 0 ? s3 : nullptr;
        if (g.f16)
            mt_layer<uint16_t>(c, x, w->layers[l], kc + l * layer_elems, vc + l * layer_elems, s1, s2, s3, add_in,
                               true);
        else
            mt_layer<float>(c, x, w->layers[l], reinterpret_cast<float*>(kc) + l * layer_elems,
                            reinterpret_cast<float*>(vc) + l * layer_elems, s1, s2, s3, add_in, true);
    }
    launch_norm(x, L > 0 ? s3 : nullptr, L > 0 ? x : nullptr, w->output_norm_w, nullptr, c.xq, g.E, g.eps, c.s,
                nullptr, T);
    mt_gemm(c, w->output_w, logits, NV, g.E);
    hipLaunchKernelGGL(k_argmax<1024>, dim3(T), dim3(1024), 0, c.s, logits, NV, nullptr, tok);
    abi_hip_ok(hipGetLastError(), fn);
}

}  // namespace
}  // namespace bpdq

extern "C" {

int generate_token(const LayerWeights* layers, const ModelConfig* cfg, const WorkBuffers* buf, const KVCache* kv,
                   int position, const void* embedding, const void* output_norm_w, const void* lm_head,
                   const void* lm_f32, int lm_K, int lm_N) {
    const char* fn = "generate_token";
    if (!bpdq::enqueue_step(bpdq::plain_opts(BPDQ_W_Q8_PAD64, cfg), layers, cfg, buf, kv, position, embedding,
                            output_norm_w, lm_head, lm_f32, lm_K, lm_N, fn))
        return -1;
    int32_t tok = -1;
    const hipStream_t s = bpdq::abi_stream();
    if (!bpdq::abi_hip_ok(hipMemcpyAsync(&tok, buf->argmax_result, 4, hipMemcpyDeviceToHost, s), fn)) return -1;
    if (!bpdq::abi_hip_ok(hipStreamSynchronize(s), fn)) return -1;
    return tok;
}

int bpd_llama_step_gpu(int weight_format, const LayerWeights* layers, const ModelConfig* cfg,
                       const WorkBuffers* buf, const KVCache* kv, int position, const void* embedding,
                       const void* output_norm_w, const void* lm_head, const void* lm_f32, int lm_K, int lm_N) {
    return bpdq::enqueue_step(bpdq::plain_opts(weight_format, cfg), layers, cfg, buf, kv, position, embedding,
                              output_norm_w, lm_head, lm_f32, lm_K, lm_N, "bpd_llama_step_gpu")
               ? 0
               : -1;
}

int bpd_llama_step_ext_gpu(int weight_format, const bpd_llama_step_opts* opts, const LayerWeights* layers,
                           const ModelConfig* cfg, const WorkBuffers* buf, const KVCache* kv, int position,
                           const void* embedding, const void* output_norm_w, const void* lm_head, const void* lm_f32,
                           int lm_K, int lm_N) {
    const char* fn = "bpd_llama_step_ext_gpu";
    bpdq::StepOpts o = bpdq::plain_opts(weight_format, cfg);
    if (opts != nullptr) {
        o.layer_formats = opts->layer_formats;
        o.lm_format = opts->lm_format < 0 ? weight_format : opts->lm_format;
        o.rope_dim = opts->rope_dim == 0 ? o.rope_dim : opts->rope_dim;
        o.rope_freqs = opts->rope_freqs;
        o.f16 = opts->kv_cache_f16 != 0;
    }
    return bpdq::enqueue_step(o, layers, cfg, buf, kv, position, embedding, output_norm_w, lm_head, lm_f32, lm_K,
                              lm_N, fn)
               ? 0
               : -1;
}

void* gpu_alloc(int bytes) {
    const char* fn = "gpu_alloc";
    if (bytes < 0) {
        bpdq::abi_error(BPDQ_ERR_SHAPE, fn, "bytes is negative");
        return nullptr;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes > 0 ? (size_t)bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        bpdq::abi_error(BPDQ_ERR_ALLOC, fn, "hipMalloc failed");
        return nullptr;
    }
    return p;
}

void bpd_llama_block_gpu(float* x, const bpd_llama_layer_weights* lw, const bpd_llama_config* cfg,
                         const int32_t* pos_ids, int n_tokens, int kv_pos, uint16_t* k_cache, uint16_t* v_cache,
                         float* scratch1, float* scratch2, float* scratch3, const float* rope_freqs) {
    bpdq::llama_block(false, x, lw, cfg, pos_ids, n_tokens, kv_pos, k_cache, v_cache, scratch1, scratch2, scratch3,
                      rope_freqs, "bpd_llama_block_gpu");
}
void bpd_llama_block_s_gpu(float* x, const bpd_llama_layer_weights* lw, const bpd_llama_config* cfg,
                           const int32_t* pos_ids, int n_tokens, int kv_pos, uint16_t* k_cache, uint16_t* v_cache,
                           float* scratch1, float* scratch2, float* scratch3, const float* rope_freqs) {
    bpdq::llama_block(true, x, lw, cfg, pos_ids, n_tokens, kv_pos, k_cache, v_cache, scratch1, scratch2, scratch3,
                      rope_freqs, "bpd_llama_block_s_gpu");
}
void bpd_llama_forward_gpu(const int32_t* token_ids, int n_tokens, const bpd_llama_weights* weights,
                           const bpd_llama_config* cfg, const int32_t* pos_ids, int kv_pos, uint16_t* k_cache,
                           uint16_t* v_cache, float* logits_out, int64_t* token_out) {
    bpdq::llama_forward(false, token_ids, n_tokens, weights, cfg, pos_ids, kv_pos, k_cache, v_cache, logits_out,
                        token_out, "bpd_llama_forward_gpu");
}
void bpd_llama_forward_s_gpu(const int32_t* token_ids, int n_tokens, const bpd_llama_weights* weights,
                             const bpd_llama_config* cfg, const int32_t* pos_ids, int kv_pos, uint16_t* k_cache,
                             uint16_t* v_cache, float* logits_out, int64_t* token_out) {
    bpdq::llama_forward(true, token_ids, n_tokens, weights, cfg, pos_ids, kv_pos, k_cache, v_cache, logits_out,
                        token_out, "bpd_llama_forward_s_gpu");
}

void gpu_free(void* p) {
    if (p != nullptr) bpdq::abi_hip_ok(hipFree(p), "gpu_free");
}

static void gpu_copy(void* dst, const void* src, int bytes, hipMemcpyKind kind, const char* fn) {
    if (bytes < 0) {
        bpdq::abi_error(BPDQ_ERR_SHAPE, fn, "bytes is negative");
        return;
    }
    if (bytes == 0) return;
    if (dst == nullptr || src == nullptr) {
        bpdq::abi_error(BPDQ_ERR_NULL, fn, "NULL pointer");
        return;
    }
    bpdq::abi_hip_ok(hipMemcpy(dst, src, (size_t)bytes, kind), fn);
}

void gpu_copy_h2d(void* dst, const void* src, int bytes) {
    gpu_copy(dst, src, bytes, hipMemcpyHostToDevice, "gpu_copy_h2d");
}
void gpu_copy_d2h(void* dst, const void* src, int bytes) {
    gpu_copy(dst, src, bytes, hipMemcpyDeviceToHost, "gpu_copy_d2h");
}
void gpu_sync(void) { bpdq::abi_hip_ok(hipDeviceSynchronize(), "gpu_sync"); }

void bpd_residual_rmsnorm_gpu(const float* x_in, const float* add, float* x_out, const float* w, float* h,
                              uint8_t* xq, int n, float eps) {
    const char* fn = "bpd_residual_rmsnorm_gpu";
    bpdq::V v{fn};
    v.need(n > 0 && n % 32 == 0 && n <= bpdq::kMaxEmbd, BPDQ_ERR_SHAPE,
           "n must be a positive multiple of 32, at most 16384");
    v.ptr(x_in, 16, "x_in");
    v.ptr(w, 16, "w");
    if (add) v.ptr(add, 16, "add");
    if (x_out) v.ptr(x_out, 16, "x_out");
    if (h) v.ptr(h, 16, "h");
    if (!v.ok || !bpdq::lds_limits_set(fn)) return;
    bpdq::launch_norm(x_in, add, x_out, w, h, xq, n, eps, bpdq::abi_stream());
    bpdq::abi_hip_ok(hipGetLastError(), fn);
}

void bpd_argmax_gpu(const float* x, int n, int32_t* out) {
    const char* fn = "bpd_argmax_gpu";
    bpdq::V v{fn};
    v.need(n > 0, BPDQ_ERR_SHAPE, "n must be positive");
    v.ptr(x, 16, "x");
    v.ptr(out, 4, "out");
    if (!v.ok) return;
    hipLaunchKernelGGL(bpdq::k_argmax<1024>, dim3(1), dim3(1024), 0, bpdq::abi_stream(), x, n, out, nullptr);
    bpdq::abi_hip_ok(hipGetLastError(), fn);
}

void bpd_expf_gpu(const float* x, float* y, int n) {
    const char* fn = "bpd_expf_gpu";
    bpdq::V v{fn};
    v.need(n >= 0, BPDQ_ERR_SHAPE, "n is negative");
    if (!v.ok || n == 0) return;
    v.ptr(x, 4, "x");
    v.ptr(y, 4, "y");
    if (!v.ok) return;
    hipLaunchKernelGGL(bpdq::k_expf, dim3((n + 255) / 256), dim3(256), 0, bpdq::abi_stream(), x, y, n);
    bpdq::abi_hip_ok(hipGetLastError(), fn);
}

}  // extern "C"
