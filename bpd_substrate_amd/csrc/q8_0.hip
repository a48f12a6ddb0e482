// q8_0.hip — Q8_0 kernels for gfx950.
//
//   k_dequant_q8_0        Q8_0 -> fp32                       (bench/bpd_cpu.c:3960-3973)
//   k_embed_q8_0          row gather + dequant               (bench/bpd_cpu.c:4002-4013)
//   k_quant_q8_0          fp32 -> Q8_0                       (bench/bpd_cpu.c:4106-4136)
//   k_q8_0_gemm_T         Q8_0 x Q8_0 cells in the AVX1 llamafile tile order
//                         (bench/bpd_gemm_q8_0_cpu.c:32-86), any number of tokens
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

// One thread per element; y = RN(float(q) * d), exact (8 x 11 bits).
__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t* __restrict__ raw, float* __restrict__ out,
                                                      int64_t n_elems) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_elems) return;
    const uint8_t* blk = raw + (i >> 5) * kQ80Bytes;
    const float d = f16_ieee((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    out[i] = (float)(int8_t)blk[2 + (i & 31)] * d;
}

void launch_dequant_q8_0(const uint8_t* raw, float* out, int n_blocks, hipStream_t s) {
    const int64_t n = (int64_t)n_blocks * 32;
    hipLaunchKernelGGL(k_dequant_q8_0, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, raw, out, n);
}

__global__ __launch_bounds__(256) void k_embed_q8_0(const uint8_t* __restrict__ table, const int32_t* __restrict__ ids,
                                                    float* __restrict__ out, int embed_dim) {
    const int t = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= embed_dim) return;
    const int64_t bpr = embed_dim / 32;
    const uint8_t* blk = table + ((int64_t)ids[t] * bpr + (e >> 5)) * kQ80Bytes;
    const float d = f16_ieee((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    out[(int64_t)t * embed_dim + e] = (float)(int8_t)blk[2 + (e & 31)] * d;
}

void launch_embed_q8_0(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_embed_q8_0, dim3((embed_dim + 255) / 256, n_tokens), dim3(256), 0, s, table, ids, out,
                       embed_dim);
}

// Q8_0 quantizer: 32 lanes per block (two blocks per wave), lane = element.
// amax is exact whatever the reduction order; d = RN(amax/127) is stored as an
// RNE binary16 (v_cvt_f16_f32); id = RN(127/amax); q = rint(RN(x*id)).
__global__ __launch_bounds__(256) void k_quant_q8_0(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                    int64_t n_blocks) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = g >> 5;
    const int e = (int)(g & 31);
    if (b >= n_blocks) return;
    const float v = x[g];
    float amax = fabsf(v);
#pragma unroll
    for (int mask = 1; mask < 32; mask <<= 1) amax = fmaxf(amax, xor_f(amax, mask));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    uint8_t* yb = y + b * kQ80Bytes;
    yb[2 + e] = (uint8_t)(int8_t)(int)__builtin_rintf(v * id);
    if (e == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);
        yb[0] = (uint8_t)(h & 0xFF);
        yb[1] = (uint8_t)(h >> 8);
    }
}

void launch_quant_q8_0(const float* x, uint8_t* y, int64_t n_elements, hipStream_t s) {
    const int64_t nb = n_elements / 32;
    const int64_t threads = nb * 32;
    hipLaunchKernelGGL(k_quant_q8_0, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, y, nb);
}

// ----------------------------------------------------------------------------
// Tile order T, one output cell per 8 lanes: lane L keeps the running fp32
// accumulator of the 4-element partial over elements 4L..4L+3 of every block,
//   acc_L = RN(RN((Ad*Bd) * float(p_L)) + acc_L)   over blocks in order,
// and the cell is ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (xor-4/2/1 butterfly).
// p_L = v_dot4_i32_i8 of the two 4-byte groups: the reference's SSSE3
// sign/maddubs/madd sequence gives the same integer for int8 values in
// [-127, 127] (it wraps only for an activation byte of -128 against a
// negative weight, which no Q8_0 quantizer produces).
// A wave holds 8 rows of one token; grid.y = tokens.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q8_0_gemm_T(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Xq,
                                                     float* __restrict__ out, int m_weight, int nb) {
    const int lane = threadIdx.x & 63;
    const int L = lane & 7;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    const int tok = blockIdx.y;
    if ((row & ~7) >= m_weight) return;
    const int rr = min(row, m_weight - 1);
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const uint8_t* wr = W + (int64_t)rr * bpr;
    const uint8_t* xr = Xq + (int64_t)tok * bpr;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = wr + (int64_t)b * kQ80Bytes;
        const uint8_t* xb = xr + (int64_t)b * kQ80Bytes;
        const uint32_t wv = ld_u32(wb + 2 + 4 * L);
        const uint32_t xv = ld_u32(xb + 2 + 4 * L);
        const float Ad = f16_ieee((uint32_t)wb[0] | ((uint32_t)wb[1] << 8));
        const float Bd = f16_ieee((uint32_t)xb[0] | ((uint32_t)xb[1] << 8));
        const float scale = Ad * Bd;
        const int p = sdot4(wv, xv, 0);
        const float prod = scale * (float)p;
        acc = prod + acc;
    }
    acc = acc + xor_f(acc, 4);
    acc = acc + xor_f(acc, 2);
    acc = acc + xor_f(acc, 1);
    if (L == 0 && row < m_weight) out[(int64_t)tok * m_weight + row] = acc;
}

void launch_q8_0_dispatch_T(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                            hipStream_t s) {
    const int nb = K / 32;
    const int waves = (m_weight + 7) / 8;
    hipLaunchKernelGGL(k_q8_0_gemm_T, dim3((waves + 3) / 4, m_tokens), dim3(256), 0, s, Wq, Xq, out, m_weight, nb);
}

}  // namespace bpdq
