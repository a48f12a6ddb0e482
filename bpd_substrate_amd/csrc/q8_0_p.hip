// q8_0_p.hip — the AVX1 build's pair order P of bpd_qdot_q8_0_q8_0_cpu
// (/root/reference/bench/bpd_cpu.c:4208-4259) for a grid of cells, and the
// entry points bpd_qdot_q8_0_q8_0_grid_gpu (and _grid_s_gpu) / bpd_qmatmul_q8_0_gpu built on it.
//
// Per output cell (weight row n, activation row m), with nb blocks:
//   8 fp32 lanes a_L = +0.0; for each block pair (2p, 2p+1), p < nb/2:
//     lane L = 4h + i takes block b = 2p + h and its elements
//     {4i..4i+3} U {16+4i..16+4i+3}: P_L = the SSSE3 sign/maddubs/madd sum of
//     those 8 products, d_b = RN(wd_b * ad_b), a_L = RN(RN(d_b * float(P_L)) + a_L);
//   s = ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7));
//   for an odd nb, the last block in the scalar form: s = RN(s + RN(float(S) * d)),
//   S its exact 32-element dot.
// P_L is the exact integer dot whenever no quant byte is -128 (|pair sums| <=
// 2*127*127 fit int16); with a -128 byte in either operand the kernel runs the
// SSSE3 arithmetic itself (|w| as an unsigned byte, y*sign(w) wrapping, int16
// saturation of each pair), so the bits match over the whole int8 range.
//
// Mapping: one cell per 8 lanes (lane = 8 r + L), a wave holds 8 weight rows of
// one activation row, grid.y = activation rows.  The activation row is staged
// once per workgroup in LDS (quant dwords, fp32 scales and a -128 flag per
// block).  Each lane's chain is serial over the nb/2 pairs, so the weight loads
// of the next U pairs are issued while the current U are accumulated.
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

namespace {

__device__ __forceinline__ uint32_t ld_u16p(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// The SSSE3 arithmetic of one dword, called only for lanes that hold a -128 byte.
__device__ __noinline__ int ssse3_quad(uint32_t w, uint32_t a) { return ssse3_quad_inl(w, a); }

// NaN cells get the bits the AVX1 reference build gives them on x86, where a NaN
// operand comes back quieted (the first operand's when both are NaN) and Inf*0,
// Inf-Inf give the default NaN.  Operand orders measured on that build with
// probes of two NaNs of different sign and payload per operand pair: the pair
// deltas d = ad*wd with the activation scale first, the lane chains
// a_L = a_L + prod with the accumulator first, the hsum as
// ((a2+a6) + (a4+a0)) + ((a3+a7) + (a5+a1)) with the left operand of each
// addition first; the odd block's delta with the weight scale first
// and s = s + prod with the sum first.  Scales decode with their payload (the
// magic-number f16 decode).  Only blocks with an Inf or NaN scale can make a lane
// non-finite, so the pairs' other blocks are skipped, 0 standing in for a finite
// lane.  Called only for a cell whose result came out NaN.
__device__ __forceinline__ float p_x86_mul(float first, float second) {
    const float r = first * second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}
__device__ __forceinline__ float p_x86_add(float first, float second) {
    const float r = first + second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}
__device__ __forceinline__ float f16_magic_dec(uint32_t h) { return f16_is_nan(h) ? f16_nan_x86(h) : f16_ieee(h); }

__device__ __forceinline__ float p_order_nan_bits(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ xrow,
                                                  int nb) {
    float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb / 2 * 2; b++) {  // the blocks of whole pairs
        const uint8_t* wb = wrow + (int64_t)b * kQ80Bytes;
        const uint8_t* xb = xrow + (int64_t)b * kQ80Bytes;
        const uint32_t hw = ld_u16p(wb), hx = ld_u16p(xb);
        if (!f16_exp31(hw) && !f16_exp31(hx)) continue;
        const float d = p_x86_mul(f16_magic_dec(hx), f16_magic_dec(hw));
        const int h = b & 1;
        for (int i = 0; i < 4; i++) {
            const int pi = ssse3_quad(ld_u32(wb + 2 + 4 * i), ld_u32(xb + 2 + 4 * i)) +
                           ssse3_quad(ld_u32(wb + 18 + 4 * i), ld_u32(xb + 18 + 4 * i));
            a[4 * h + i] = p_x86_add(a[4 * h + i], p_x86_mul(d, (float)pi));
        }
    }
    const float l0 = p_x86_add(a[4], a[0]), l1 = p_x86_add(a[2], a[6]);
    const float l2 = p_x86_add(a[5], a[1]), l3 = p_x86_add(a[3], a[7]);
    float s = p_x86_add(p_x86_add(l1, l0), p_x86_add(l3, l2));
    if (nb & 1) {
        const uint8_t* wb = wrow + (int64_t)(nb - 1) * kQ80Bytes;
        const uint8_t* xb = xrow + (int64_t)(nb - 1) * kQ80Bytes;
        int sumi = 0;
        for (int j = 0; j < 32; j++) sumi += (int)(int8_t)wb[2 + j] * (int)(int8_t)xb[2 + j];
        const float d = p_x86_mul(f16_magic_dec(ld_u16p(wb)), f16_magic_dec(ld_u16p(xb)));
        s = p_x86_add(s, p_x86_mul((float)sumi, d));
    }
    return s;
}

template <int U>
struct PBatch {
    uint32_t q0[U], q1[U];  // weight dwords i and 4+i of block 2p+h
    uint32_t d[U];          // its scale (binary16 bits)
};

template <int U>
__device__ __forceinline__ void p_load(PBatch<U>& w, const uint8_t* __restrict__ wbase, uint32_t voff, uint32_t doff,
                                       int h, int p0, int np) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        // pairs past the end repeat the last pair (their steps are skipped)
        const uint8_t* bu = wbase + (int64_t)(2 * min(p0 + u, np - 1) + h) * kQ80Bytes;
        w.q0[u] = ld_u32(bu + voff);
        w.q1[u] = ld_u32(bu + voff + 16);
        w.d[u] = ld_u16p(bu + doff);
    }
}

template <int U>
__device__ __forceinline__ float p_accumulate(const PBatch<U>& w, const uint32_t* __restrict__ xs,
                                              const float* __restrict__ xd, const uint32_t* __restrict__ xf, int h,
                                              int i, int p0, int np, float acc) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int p = p0 + u;
        if (p < np) {
            const int b = 2 * p + h;
            const uint32_t x0 = xs[b * 8 + i], x1 = xs[b * 8 + 4 + i];
            int pv = sdot4(w.q1[u], x1, sdot4(w.q0[u], x0, 0));
            if (xf[b] | has_m128(w.q0[u]) | has_m128(w.q1[u])) pv = ssse3_quad(w.q0[u], x0) + ssse3_quad(w.q1[u], x1);
            const float delta = f16_ieee(w.d[u]) * xd[b];
            const float prod = delta * (float)pv;
            acc = prod + acc;
        }
    }
    return acc;
}

// The activation row into LDS: xs[b*8 + j] = quant dword j of block b, xd[b] its
// scale as fp32, xf[b] nonzero when one of its quants is -128.
template <int NT>
__device__ __forceinline__ void p_stage_x(uint32_t* __restrict__ xs, float* __restrict__ xd, uint32_t* __restrict__ xf,
                                          const uint8_t* __restrict__ xr, int nb) {
    for (int b = threadIdx.x; b < nb; b += NT) xf[b] = 0;
    __syncthreads();
    const int n = nb * 8;
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * NT) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(i0 + u * NT, n - 1);
            v[u] = ld_u32(xr + (int64_t)(i >> 3) * kQ80Bytes + 2 + 4 * (i & 7));
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * NT;
            if (i < n) {
                xs[i] = v[u];
                if (has_m128(v[u])) xf[i >> 3] = 1;
            }
        }
    }
    for (int b = threadIdx.x; b < nb; b += NT) xd[b] = f16_ieee(ld_u16p(xr + (int64_t)b * kQ80Bytes));
}

template <int U, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q8_0_qdot_P(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Xq,
                                                          float* __restrict__ out, int n_rows, int nb) {
    extern __shared__ uint32_t lds[];
    uint32_t* xs = lds;                                  // [nb][8]
    float* xd = reinterpret_cast<float*>(lds + nb * 8);  // [nb]
    uint32_t* xf = lds + nb * 9;                         // [nb]
    const int lane = threadIdx.x & 63, L = lane & 7, h = L >> 2, i = L & 3;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = (blockIdx.x * WPB + wave) * 8 + (lane >> 3);
    const int tok = blockIdx.y;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    // spare waves and rows read row n_rows-1 (nothing is stored for them)
    const int row0 = min((blockIdx.x * WPB + wave) * 8, n_rows - 1);
    const uint8_t* wbase = W + (int64_t)row0 * bpr;
    const uint32_t doff = (uint32_t)((max(min(row, n_rows - 1), row0) - row0) * bpr);
    const uint32_t voff = doff + 2 + 4 * i;
    const int np = nb / 2;

    PBatch<U> a, b;
    if (np > 0) p_load<U>(a, wbase, voff, doff, h, 0, np);
    p_stage_x<64 * WPB>(xs, xd, xf, Xq + (int64_t)tok * bpr, nb);
    __syncthreads();

    float acc = 0.0f;
    for (int p0 = 0; p0 < np; p0 += 2 * U) {
        if (p0 + U < np) p_load<U>(b, wbase, voff, doff, h, p0 + U, np);
        acc = p_accumulate<U>(a, xs, xd, xf, h, i, p0, np, acc);
        if (p0 + 2 * U < np) p_load<U>(a, wbase, voff, doff, h, p0 + 2 * U, np);
        acc = p_accumulate<U>(b, xs, xd, xf, h, i, p0 + U, np, acc);
    }
    // lane L pairs with L^4, then L^2, then L^1: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))
    acc = acc + xor_f(acc, 4);
    acc = acc + xor_f(acc, 2);
    acc = acc + xor_f(acc, 1);
    if (nb & 1) {  // the odd last block, scalar form: exact 32-element dot, one product, one add
        const int bl = nb - 1;
        const uint8_t* wl = wbase + doff + (int64_t)bl * kQ80Bytes;
        int s = sdot4(ld_u32(wl + 2 + 4 * L), xs[bl * 8 + L], 0);
        s += xor_i(s, 4);
        s += xor_i(s, 2);
        s += xor_i(s, 1);
        acc = acc + (float)s * (f16_ieee(ld_u16p(wl)) * xd[bl]);
    }
    if (L == 0 && row < n_rows) {
        if (__builtin_isnan(acc)) acc = p_order_nan_bits(W + (int64_t)row * bpr, Xq + (int64_t)tok * bpr, nb);
        out[(int64_t)tok * n_rows + row] = acc;
    }
}

}  // namespace

// LDS of the staged activation row: nb * 40 bytes (up to K = 52,416 in 64 KB).
int qdot_p_max_k() { return (64 * 1024 / 40) / 2 * 2 * 32; }

void launch_q8_0_qdot_P(const uint8_t* Wq, const uint8_t* Xq, float* out, int n_rows, int m_tokens, int K,
                        hipStream_t s) {
    const int nb = K / 32;
    if (nb == 0) {  // every cell is the empty sum
        launch_fill_zero(out, (int64_t)n_rows * m_tokens, s);
        return;
    }
    constexpr int U = 8, WPB = 4;
    const int waves = (n_rows + 7) / 8;
    const size_t lds = (size_t)nb * 40;
    hipLaunchKernelGGL((k_q8_0_qdot_P<U, WPB>), dim3((waves + WPB - 1) / WPB, m_tokens), dim3(64 * WPB), lds, s, Wq,
                       Xq, out, n_rows, nb);
}

}  // namespace bpdq
