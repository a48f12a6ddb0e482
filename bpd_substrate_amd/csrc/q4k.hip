// q4k.hip — Q4_K super-block kernels for gfx950.
//
//   k_dequant_q4k<ORDER>   Q4_K -> fp32, bpd element map or GGUF element map
//   k_qmatmul_q4k_chain    reference-order GEMV with fp32 x (one fp32 chain per row)
//   k_quant_q8k            fp32 -> Q8_K activation blocks
//   k_q4k_q8k_gemv<ORDER,R> Q4_K x Q8_K GEMV, integer sub-block sums + fixed fp32 tree
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

// ----------------------------------------------------------------------------
// Dequant.  One wave per Q4_K block; lane l writes elements 4l..4l+3, so each
// wave store is one contiguous 1 KB line of output.  The four elements come
// from the low or the high nibbles of one qs dword:
//   bpd map  (bench/bpd_quant.c:68-72): sub-block j = l/8, qs dword 4j + l%4,
//            high nibbles when bit 2 of l is set
//   GGUF map (bench_dequant_gpu_h2h.cu:31-46): group i = l/16, qs dword 8i + l%8,
//            high nibbles (sub-block 2i+1) when bit 3 of l is set, else sub-block 2i
// y = RN(d*sc*q - dmin*m): d*sc and (d*sc)*q are exact in fp32, so
// fmaf(d*sc, q, -dmin*m) equals the reference's multiply-then-subtract bit for bit.
// The output is written with non-temporal stores: nothing re-reads it here, and
// skipping the cache allocation lifts the write stream from ~4.7 to ~6.4 TB/s.
// ----------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int ORDER>
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ q, float* __restrict__ out,
                                                     int n_blocks) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= n_blocks) return;
    int dw, j, hi;
    if (ORDER == 0) {
        j = lane >> 3;
        dw = 4 * j + (lane & 3);
        hi = (lane >> 2) & 1;
    } else {
        const int i = lane >> 4;
        dw = 8 * i + (lane & 7);
        hi = (lane >> 3) & 1;
        j = 2 * i + hi;
    }
    const uint8_t* blk = q + b * kQ4KBytes;
    const uint4 hdr = ld_u128(blk);
    const uint32_t qw = ld_u32(blk + 16 + 4 * dw);
    const float d = ORDER == 0 ? f16_ieee(hdr.x) : f16_h2h(hdr.x);
    const float dmin = ORDER == 0 ? f16_ieee(hdr.x >> 16) : f16_h2h(hdr.x >> 16);
    int sc, m;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
    const float s = d * (float)sc, mn = dmin * (float)m;
    const uint32_t nib = (hi ? (qw >> 4) : qw) & 0x0F0F0F0Fu;
    f32x4 v;
    v.x = fmaf(s, (float)(nib & 0xFFu), -mn);
    v.y = fmaf(s, (float)((nib >> 8) & 0xFFu), -mn);
    v.z = fmaf(s, (float)((nib >> 16) & 0xFFu), -mn);
    v.w = fmaf(s, (float)(nib >> 24), -mn);
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + b * 256 + 4 * lane));
}

void launch_dequant_q4k(const uint8_t* q, float* out, int n_blocks, int order, hipStream_t s) {
    const dim3 grid((unsigned)(((int64_t)n_blocks + 3) / 4));
    if (order == 0)
        hipLaunchKernelGGL(k_dequant_q4k<0>, grid, dim3(256), 0, s, q, out, n_blocks);
    else
        hipLaunchKernelGGL(k_dequant_q4k<1>, grid, dim3(256), 0, s, q, out, n_blocks);
}

// ----------------------------------------------------------------------------
// Reference-order GEMV with fp32 x (bench/bpd_quant.c:88-109): one lane per row
// runs y = (((0 + w0*x0) + w1*x1) + ...) over k in bpd element order, each
// product and each sum rounded once.  Rows are independent, so this is
// bit-identical to the CPU reference; the chain itself is serial by definition.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_qmatmul_q4k_chain(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int nb) {
    const int row = blockIdx.x * 64 + threadIdx.x;
    if (row >= M) return;
    const uint8_t* rp = w + (int64_t)row * nb * kQ4KBytes;
    float sum = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = rp + (int64_t)b * kQ4KBytes;
        const uint4 hdr = ld_u128(blk);
        const float d = f16_ieee(hdr.x), dmin = f16_ieee(hdr.x >> 16);
        const float* xb = x + (int64_t)b * 256;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
            const float scale = d * (float)sc, mn = dmin * (float)m;
            const uint4 qv = ld_u128(blk + 16 + 16 * j);
            const uint32_t qd[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float v = fmaf(scale, (float)((qd[k >> 2] >> (8 * (k & 3))) & 15u), -mn);
                sum = sum + v * xb[32 * j + k];
            }
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float v = fmaf(scale, (float)((qd[k >> 2] >> (8 * (k & 3) + 4)) & 15u), -mn);
                sum = sum + v * xb[32 * j + 16 + k];
            }
        }
    }
    y[row] = sum;
}

void launch_qmatmul_q4k_chain(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t s) {
    hipLaunchKernelGGL(k_qmatmul_q4k_chain, dim3((M + 63) / 64), dim3(64), 0, s, w, x, y, M, K / 256);
}

// ----------------------------------------------------------------------------
// Q8_K quantizer: one wave per 256-element block, lane l holds elements 4l..4l+3.
// d = RN(amax/127), id = amax ? RN(127/amax) : 0, q = rint(RN(x*id)),
// bsums[g] = sum of q[16g..16g+15] (lanes 4g..4g+3).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_q8k(const float* __restrict__ x, uint8_t* __restrict__ y, int nb) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;
    const float4 v = *reinterpret_cast<const float4*>(x + (int64_t)b * 256 + 4 * lane);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int mask = 1; mask < 64; mask <<= 1) amax = fmaxf(amax, xor_f(amax, mask));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q0 = (int)__builtin_rintf(v.x * id), q1 = (int)__builtin_rintf(v.y * id);
    const int q2 = (int)__builtin_rintf(v.z * id), q3 = (int)__builtin_rintf(v.w * id);
    uint8_t* yb = y + (int64_t)b * kQ8KBytes;
    const uint32_t packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
                            ((uint32_t)(q3 & 0xFF) << 24);
    *reinterpret_cast<uint32_t*>(yb + 4 + 4 * lane) = packed;
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<0xB1>(s);
    s += dpp_i<0x4E>(s);
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(yb + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *reinterpret_cast<float*>(yb) = d;
}

void launch_quant_q8k(const float* x, uint8_t* y, int n, hipStream_t s) {
    const int nb = n / 256;
    hipLaunchKernelGGL(k_quant_q8k, dim3((nb + 3) / 4), dim3(256), 0, s, x, y, nb);
}

// ----------------------------------------------------------------------------
// Q4_K x Q8_K GEMV.  A wave covers R rows.  Lane (q = lane/8, c = lane%8) owns
// qs bytes 16c..16c+15 of super-block 8t+q in every block-group t: one 16-B load
// per lane, so a wave instruction reads the qs of 8 consecutive super-blocks.
//   bpd map: those 16 bytes are exactly sub-block c (low nibbles with x[32c+k],
//            high nibbles with x[32c+16+k]).
//   GGUF map: low nibbles are elements 64(c/2)+16(c%2)+k of sub-block 2(c/2),
//            high nibbles the same +32, of sub-block 2(c/2)+1.
// Integer partials are summed exactly over the 8 lanes of a super-block; the
// fp32 combine and the per-row tree are the fixed order documented in
// the C restatement: slot sums s_q from +0.0 over b = q mod 8 ascending, then
// ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)) as an xor-8/16/32 butterfly.
// ----------------------------------------------------------------------------
// Per-lane activation operands of one super-block: the 32 q8 values that meet
// this lane's 32 nibbles, the lane's pair of bsums, and the block scale.
struct XOps {
    uint32_t lo[4], hi[4];
    int bsum;
    float dy;
};

// x operands of one super-block for lane c (xb = the Q8_K block).
template <int ORDER>
__device__ __forceinline__ XOps load_x(const uint8_t* __restrict__ xb, int c) {
    XOps o;
    o.dy = *reinterpret_cast<const float*>(xb);
    const uint32_t bs = ld_u32(xb + 260 + 4 * c);
    o.bsum = (int)(int16_t)(bs & 0xFFFFu) + (int)(int16_t)(bs >> 16);
    const int off_lo = ORDER == 0 ? 32 * c : 64 * (c >> 1) + 16 * (c & 1);
    const int off_hi = ORDER == 0 ? 32 * c + 16 : off_lo + 32;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o.lo[k] = ld_u32(xb + 4 + off_lo + 4 * k);
        o.hi[k] = ld_u32(xb + 4 + off_hi + 4 * k);
    }
    return o;
}

// The 16 header bytes {d, dmin, scales[12]} of a super-block: lane c of a slot
// loaded dword (c & 3); four quad broadcasts give every lane all four dwords.
__device__ __forceinline__ uint4 bcast_header(uint32_t mine) {
    uint4 h;
    h.x = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0x00, 0xF, 0xF, false);  // quad_perm [0,0,0,0]
    h.y = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0x55, 0xF, 0xF, false);  // quad_perm [1,1,1,1]
    h.z = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xAA, 0xF, 0xF, false);  // quad_perm [2,2,2,2]
    h.w = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xFF, 0xF, 0xF, false);  // quad_perm [3,3,3,3]
    return h;
}

// Contribution c_b of one super-block (same value in all 8 lanes of the slot).
// |S| <= 32*15*127 and sc, m <= 63, so the 24-bit multiplies are exact.
template <int ORDER>
__device__ __forceinline__ float block_contrib(const uint4& hdr, const uint4& qv, const XOps& x, int c) {
    const uint32_t qd[4] = {qv.x, qv.y, qv.z, qv.w};
    int s_lo = 0, s_hi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        s_lo = sdot4(qd[k] & 0x0F0F0F0Fu, x.lo[k], s_lo);
        s_hi = sdot4((qd[k] >> 4) & 0x0F0F0F0Fu, x.hi[k], s_hi);
    }
    int sc, m, isum;
    if (ORDER == 0) {
        q4k_scale_min(hdr.y, hdr.z, hdr.w, c, sc, m);
        isum = __mul24(sc, s_lo + s_hi);
    } else {
        int sc2, m2;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1), sc, m2);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1) + 1, sc2, m2);
        isum = __mul24(sc, s_lo) + __mul24(sc2, s_hi);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, c, sc2, m);
    }
    int msum = __mul24(m, x.bsum);
    isum = sum8_i(isum);
    msum = sum8_i(msum);
    const float dd = f16_ieee(hdr.x) * x.dy;
    const float dm = f16_ieee(hdr.x >> 16) * x.dy;
    const float a = dd * (float)isum;
    const float mm = dm * (float)msum;
    return a - mm;
}

// One wave's R rows: each pass issues the loads of G block-groups x R rows (a
// 16-byte qs load and a header dword per lane each) before computing any of
// them, so every wave keeps its whole share of the stream in flight.  Rows past
// M reuse row M-1 and slots past nb reuse block nb-1 (their results are
// discarded), so every address stays in the tensors.  row0 < M.
template <int ORDER, int R, int G>
__device__ __forceinline__ void gemv_rows(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xq,
                                          float* __restrict__ y, int M, int nb, int row0) {
    const int lane = threadIdx.x & 63;
    const int q = lane >> 3, c = lane & 7;
    const int64_t row_bytes = (int64_t)nb * kQ4KBytes;
    const int ngroups = (nb + 7) >> 3;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;

    for (int t0 = 0; t0 < ngroups; t0 += G) {
        uint32_t hw[G][R];
        uint4 qv[G][R];
        XOps x[G];
        bool valid[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int b = (t0 + g) * 8 + q;
            valid[g] = b < nb;
            const int bb = valid[g] ? b : nb - 1;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t* blk = w + (int64_t)min(row0 + r, M - 1) * row_bytes + (int64_t)bb * kQ4KBytes;
                qv[g][r] = ld_u128(blk + 16 + 16 * c);
                hw[g][r] = ld_u32(blk + 4 * (c & 3));
            }
            x[g] = load_x<ORDER>(xq + (int64_t)bb * kQ8KBytes, c);
        }
        // every load of the pass is issued before any of its data is used
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float cb = block_contrib<ORDER>(bcast_header(hw[g][r]), qv[g][r], x[g], c);
                if (valid[g]) s[r] = s[r] + cb;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        float v = s[r];
        v = v + xor_f(v, 8);
        v = v + xor_f(v, 16);
        v = v + xor_f(v, 32);
        if (lane == 0 && row0 + r < M) y[row0 + r] = v;
    }
}

// R rows per wave, WPB waves per workgroup.
template <int ORDER, int R, int G, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_gemv(const uint8_t* __restrict__ w,
                                                           const uint8_t* __restrict__ xq, float* __restrict__ y,
                                                           int M, int nb) {
    // the wave index is uniform across the wave; saying so keeps row offsets scalar
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (blockIdx.x * WPB + wave) * R;
    if (row0 >= M) return;
    gemv_rows<ORDER, R, G>(w, xq, y, M, nb, row0);
}

// Up to kMulti matrices that share one activation vector (Q/K/V, gate/up) in
// one launch: waves are numbered across the matrices, matrix i owning waves
// [first[i], first[i+1]).  Each row is computed exactly as the single-matrix
// kernel computes it.
constexpr int kMulti = 4;
struct MultiArgs {
    const uint8_t* w[kMulti];
    float* y[kMulti];
    int M[kMulti];
    int first[kMulti + 1];
};

template <int ORDER, int R, int G, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_gemv_multi(MultiArgs a, const uint8_t* __restrict__ xq, int nb) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int gw = blockIdx.x * WPB + wave;
    int i = 0;
#pragma unroll
    for (int k = 1; k < kMulti; k++)
        if (gw >= a.first[k]) i = k;
    if (gw >= a.first[kMulti]) return;
    const int row0 = (gw - a.first[i]) * R;
    if (row0 >= a.M[i]) return;
    gemv_rows<ORDER, R, G>(a.w[i], xq, a.y[i], a.M[i], nb, row0);
}

template <int ORDER, int R, int G, int WPB>
static void launch_gemv(const uint8_t* w, const uint8_t* xq, float* y, int M, int nb, hipStream_t s) {
    const int waves = (M + R - 1) / R;
    hipLaunchKernelGGL((k_q4k_q8k_gemv<ORDER, R, G, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0, s, w,
                       xq, y, M, nb);
}

template <int ORDER>
static void launch_gemv_order(const uint8_t* w, const uint8_t* xq, float* y, int M, int nb, hipStream_t s) {
    const int ngroups = (nb + 7) / 8;
    // shapes measured on MI355X: 2 rows x 2 block-groups per pass; wider
    // workgroups pay off when the row is long (several passes per wave)
    if (ngroups <= 2)
        launch_gemv<ORDER, 2, 2, 4>(w, xq, y, M, nb, s);
    else
        launch_gemv<ORDER, 2, 2, 8>(w, xq, y, M, nb, s);
}

void launch_qmatmul_q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s) {
    const int nb = K / 256;
    if (order == 0)
        launch_gemv_order<0>(w, xq, y, M, nb, s);
    else
        launch_gemv_order<1>(w, xq, y, M, nb, s);
}

template <int ORDER, int WPB>
static void launch_multi(const MultiArgs& a, const uint8_t* xq, int nb, hipStream_t s) {
    const int waves = a.first[kMulti];
    hipLaunchKernelGGL((k_q4k_q8k_gemv_multi<ORDER, 2, 2, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0, s,
                       a, xq, nb);
}

void launch_qmatmul_q4k_q8k_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const uint8_t* xq,
                                  int K, int order, hipStream_t s) {
    constexpr int R = 2;
    MultiArgs a;
    int waves = 0;
    for (int i = 0; i < kMulti; i++) {
        const bool used = i < n;
        a.w[i] = used ? w[i] : nullptr;
        a.y[i] = used ? y[i] : nullptr;
        a.M[i] = used ? M[i] : 0;
        a.first[i] = waves;
        waves += used ? (M[i] + R - 1) / R : 0;
    }
    a.first[kMulti] = waves;
    if (waves == 0) return;
    const int nb = K / 256;
    const bool long_rows = (nb + 7) / 8 > 2;
    if (order == 0) {
        if (long_rows) launch_multi<0, 8>(a, xq, nb, s); else launch_multi<0, 4>(a, xq, nb, s);
    } else {
        if (long_rows) launch_multi<1, 8>(a, xq, nb, s); else launch_multi<1, 4>(a, xq, nb, s);
    }
}

}  // namespace bpdq
