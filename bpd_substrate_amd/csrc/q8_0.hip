// q8_0.hip — Q8_0 kernels for gfx950.
//
//   k_dequant_q8_0        Q8_0 -> fp32                       (bench/bpd_cpu.c:3960-3973)
//   k_embed_q8_0          row gather + dequant               (bench/bpd_cpu.c:4002-4013)
//   k_quant_q8_0          fp32 -> Q8_0                       (bench/bpd_cpu.c:4106-4136)
//   k_q8_0_gemv_T         Q8_0 x Q8_0 cells in the AVX1 llamafile tile order
//                         (bench/bpd_gemm_q8_0_cpu.c:32-86), pipelined chains
//   k_q8_0_gemv_TP        the same cells, block products by producer waves and the
//                         chains from LDS (few rows, long rows)
//   k_q8_0_gemv_V         the same cells, each wave streaming its 2 rows as 16-byte
//                         lanes through its own LDS slot, four lanes per chain
//   k_q8_0_gemm_T         the same cells, plain, for rows too long to stage
//   k_q8_pad64            fp32 -> the padded Q8 layout (inference/llamatov_c_inference.py:88-100)
//   k_q8_0_gemm_S(H)      the scalar order S on int8 MFMA (prefill)
#include <mutex>

#include "bpdq_device.h"
#include "bpdq_launch.h"
#include "bpdq_math.h"

namespace bpdq {

// One thread per element; y = RN(float(q) * d), exact (8 x 11 bits).
__global__ __launch_bounds__(256) void k_dequant_q8_0(const uint8_t* __restrict__ raw, float* __restrict__ out,
                                                      int64_t n_elems) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_elems) return;
    const uint8_t* blk = raw + (i >> 5) * kQ80Bytes;
    const uint32_t hd = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
    out[i] = mul_nan_x86((float)(int8_t)blk[2 + (i & 31)] * f16_ieee(hd), hd);
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
    const uint32_t hd = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
    out[(int64_t)t * embed_dim + e] = mul_nan_x86((float)(int8_t)blk[2 + (e & 31)] * f16_ieee(hd), hd);
}

void launch_embed_q8_0(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_embed_q8_0, dim3((embed_dim + 255) / 256, n_tokens), dim3(256), 0, s, table, ids, out,
                       embed_dim);
}

// Q8_0 quantizer: 32 lanes per block (two blocks per wave), lane = element
// (q8_0_lane_store).
__global__ __launch_bounds__(256) void k_quant_q8_0(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                    int64_t n_blocks) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = g >> 5;
    if (b >= n_blocks) return;
    q8_0_lane_store(x[g], y + b * kQ80Bytes, (int)(g & 31));
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
//
// The chain over blocks is serial, so the kernel hides memory latency by
// software pipelining: each lane prefetches the weight dword and scale of the
// next U blocks while it accumulates the current U.  The token's activation row
// is staged once per workgroup in LDS, its 32 quants 4-byte aligned per block
// and its scale decoded to fp32, so each step reads x with two LDS broadcasts.
// ----------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// ----------------------------------------------------------------------------
// Cells of the AVX1 tile order T (bench/bpd_gemm_q8_0_cpu.c:32-86) that the fast
// kernels below cannot give bit for bit are recomputed by one lane in the
// reference's own arithmetic (t_order_cell): NaN cells, and every cell of an
// activation row holding a -128 quant (where SSSE3's sign/maddubs wrap: -(-128)
// is -128 against a negative weight; the kernels use the exact dot, which the
// Q8_0 quantizers' [-127, 127] output always gives).  NaN bits: the reference build
// on x86 gives a NaN operand back
// quieted (the first operand's when both are NaN) and Inf*0, Inf-Inf give the
// default NaN.  Which operand is first differs between the build's nine tile
// kernels, so a cell's bits depend on the tile that computes it
// (bench/bpd_gemm_q8_0_cpu.c:159-207: tiles of 4, then 2, then 1 rows and
// tokens).  Measured on that build, one probe per operand pair with NaNs of both
// signs: Ad and Bd come from the ldexpf decode of :13-26 (an f16 NaN becomes
// +/-0x7FC00000, no payload); scale = Bd*Ad with Bd first in every tile; lane L's
// product scale*float(p_L); its chain acc_L = prod + acc_L with the accumulator
// first in the 1x1 tile and the product first in the others; the hsum
// ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)) with a per-cell mask of swapped additions
// (t_tile_mask).  Weight block b of the row is at wrow + b * bstride, its quants
// at +qoff.
// ----------------------------------------------------------------------------
__device__ __forceinline__ float x86_mul(float first, float second) {
    const float r = first * second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}
__device__ __forceinline__ float x86_add(float first, float second) {
    const float r = first + second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}
__device__ __forceinline__ float x86_add_sw(float a, float b, uint32_t sw) { return sw ? x86_add(b, a) : x86_add(a, b); }
__device__ __forceinline__ float f16_tile(uint32_t h) {
    if (!f16_is_nan(h)) return f16_ieee(h);
    return __uint_as_float(((h & 0x8000u) << 16) | 0x7FC00000u);
}

// The tile of cell (row r, token t) and its hsum mask: bits 0-3 swap the pairs
// (a0,a4), (a2,a6), (a1,a5), (a3,a7) (the right one first), bit 4 the left
// second-level sum, bit 5 the right one, bit 6 the top addition.  *acc_first:
// the 1x1 tile.
__device__ __forceinline__ uint32_t t_tile_mask(int r, int t, int m_weight, int m_tokens, bool* acc_first) {
    const int full_r = m_weight / 4 * 4, full_t = m_tokens / 4 * 4;
    const int RM = r < full_r ? 4 : (m_weight - full_r >= 2 && r < full_r + 2) ? 2 : 1;
    const int RN = t < full_t ? 4 : (m_tokens - full_t >= 2 && t < full_t + 2) ? 2 : 1;
    const int i = RM == 4 ? r % 4 : RM == 2 ? r - full_r : 0;
    const int j = RN == 4 ? t % 4 : RN == 2 ? t - full_t : 0;
    *acc_first = RM == 1 && RN == 1;
    if (RM == 4) return 0x12u;
    if (RM == 2) return (RN == 1 || i == 0) ? 0u : 0x12u;
    return RN == 4 ? 0x10u : RN == 2 ? (j == 0 ? 0x01u : 0x10u) : 0u;
}

__device__ __forceinline__ float t_order_cell(const uint8_t* __restrict__ wrow, int64_t bstride, int qoff,
                                             const uint8_t* __restrict__ xrow, int nb, int r, int t, int m_weight,
                                             int m_tokens) {
    bool acc_first;
    const uint32_t m = t_tile_mask(r, t, m_weight, m_tokens, &acc_first);
    float C[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = wrow + (int64_t)b * bstride;
        const uint8_t* xb = xrow + (int64_t)b * kQ80Bytes;
        const uint32_t hw = (uint32_t)wb[0] | ((uint32_t)wb[1] << 8);
        const uint32_t hx = (uint32_t)xb[0] | ((uint32_t)xb[1] << 8);
        const float scale = x86_mul(f16_tile(hx), f16_tile(hw));
#pragma unroll
        for (int L = 0; L < 8; L++) {
            const int p = ssse3_quad_inl(ld_u32(wb + qoff + 4 * L), ld_u32(xb + 2 + 4 * L));
            const float prod = x86_mul(scale, (float)p);
            C[L] = acc_first ? x86_add(C[L], prod) : x86_add(prod, C[L]);
        }
    }
    const float l0 = x86_add_sw(C[0], C[4], m & 1u), l1 = x86_add_sw(C[2], C[6], m & 2u);
    const float l2 = x86_add_sw(C[1], C[5], m & 4u), l3 = x86_add_sw(C[3], C[7], m & 8u);
    return x86_add_sw(x86_add_sw(l0, l1, m & 16u), x86_add_sw(l2, l3, m & 32u), m & 64u);
}

// Whether the activation row holds a -128 quant: the waves of the workgroup record
// theirs in wave_m128[wave] while staging (every wave writes its entry, so no
// clearing is needed), read after the staging barrier.
__device__ __forceinline__ void note_m128(uint32_t* wave_m128, uint32_t any_m128) {
    const bool w = __ballot(any_m128 != 0) != 0;
    if ((threadIdx.x & 63) == 0) wave_m128[threadIdx.x >> 6] = w ? 1u : 0u;
}
__device__ __forceinline__ bool row_m128(const uint32_t* wave_m128, int nwaves) {
    uint32_t a = 0;
    for (int i = 0; i < nwaves; i++) a |= wave_m128[i];
    return a != 0;
}

template <int U>
struct WBatch {
    uint32_t q[U];   // weight bytes 2+4L..5+4L of block b
    uint32_t d[U];   // weight scale (binary16 bits) of block b
};

// wbase: wave-uniform pointer to the wave's first row; voff: this lane's row
// offset within the wave plus 2 + 4L (lane-constant).  Addresses are then
// "scalar base + 32-bit lane offset + immediate", one instruction per load.
template <int U, int LAYOUT>
__device__ __forceinline__ void load_batch(WBatch<U>& w, const uint8_t* __restrict__ wbase, uint32_t voff,
                                           uint32_t doff, int b0, int nb, int64_t bstride) {
    // Blocks past the end of the row repeat block nb-1 (their steps are skipped).
    // The clamp is wave-uniform, so each address stays scalar base + lane offset.
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint8_t* bu = wbase + (int64_t)min(b0 + u, nb - 1) * (LAYOUT == 0 ? (int64_t)kQ80Bytes : bstride);
        w.q[u] = ld_u32(bu + voff);
        w.d[u] = ld_u16(bu + doff);
    }
}

template <int U>
__device__ __forceinline__ float accumulate_batch(const WBatch<U>& w, const uint32_t* __restrict__ xs,
                                                  const float* __restrict__ xd, int L, int b0, int nb, float acc) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int b = b0 + u;
        if (b < nb) {
            const float scale = f16_ieee(w.d[u]) * xd[b];
            const int p = sdot4(w.q[u], xs[b * 8 + L], 0);
            const float prod = scale * (float)p;
            acc = prod + acc;
        }
    }
    return acc;
}

// The token's activation row into LDS: xs[b*8 + L] = quant dword L of block b,
// xd[b] = its scale as fp32.  Each pass issues all its loads (8 per thread)
// before storing any, so staging costs one memory latency per 8*NT dwords
// instead of one per loop trip.
template <int NT>
__device__ __forceinline__ uint32_t stage_x(uint32_t* __restrict__ xs, float* __restrict__ xd,
                                            const uint8_t* __restrict__ xr, int nb) {
    const int n = nb * 8;
    uint32_t any_m128 = 0;
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * NT) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(i0 + u * NT, n - 1);
            v[u] = ld_u32(xr + (int64_t)(i >> 3) * kQ80Bytes + 2 + 4 * (i & 7));
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + u * NT < n) {
                xs[i0 + u * NT] = v[u];
                any_m128 |= has_m128(v[u]);
            }
    }
    for (int i0 = threadIdx.x; i0 < nb; i0 += 8 * NT) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = ld_u16(xr + (int64_t)min(i0 + u * NT, nb - 1) * kQ80Bytes);
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + u * NT < nb) xd[i0 + u * NT] = f16_ieee(v[u]);
    }
    return any_m128;
}

// LAYOUT 0: W is rows of 34-byte Q8_0 blocks.  LAYOUT 1: W is the padded
// block-major layout of inference/llamatov_c_inference.py:88-100, records of 64
// bytes [block][row] with d at bytes 0-1 and the quants at 4-35; the cells and
// their order are the same.
template <int U, int WPB, int LAYOUT = 0>
__global__ __launch_bounds__(64 * WPB) void k_q8_0_gemv_T(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Xq,
                                                          float* __restrict__ out, int m_weight, int nb) {
    extern __shared__ uint32_t lds[];
    uint32_t* xs = lds;                                   // [nb][8] activation quants
    float* xd = reinterpret_cast<float*>(lds + nb * 8);   // [nb] activation scales
    const int lane = threadIdx.x & 63;
    const int L = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = (blockIdx.x * WPB + wave) * 8 + (lane >> 3);
    const int tok = blockIdx.y;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const int64_t wrow = LAYOUT == 0 ? bpr : 64, bstride = LAYOUT == 0 ? kQ80Bytes : (int64_t)m_weight * 64;
    // A wave past the last row (the workgroup's spare waves) reads row m_weight-1;
    // base and lane offsets are clamped so every address stays inside W.
    const int row0 = min((blockIdx.x * WPB + wave) * 8, m_weight - 1);
    const uint8_t* wbase = W + (int64_t)row0 * wrow;
    const uint32_t doff = (uint32_t)((max(min(row, m_weight - 1), row0) - row0) * wrow);
    const uint32_t voff = doff + (LAYOUT == 0 ? 2 : 4) + 4 * L;

    __shared__ uint32_t wave_m128[WPB];
    WBatch<U> a, b;
    load_batch<U, LAYOUT>(a, wbase, voff, doff, 0, nb, bstride);
    note_m128(wave_m128, stage_x<64 * WPB>(xs, xd, Xq + (int64_t)tok * bpr, nb));
    __syncthreads();
    const bool xm128 = __builtin_amdgcn_readfirstlane((int)row_m128(wave_m128, WPB)) != 0;

    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 2 * U) {
        if (b0 + U < nb) load_batch<U, LAYOUT>(b, wbase, voff, doff, b0 + U, nb, bstride);
        acc = accumulate_batch<U>(a, xs, xd, L, b0, nb, acc);
        if (b0 + 2 * U < nb) load_batch<U, LAYOUT>(a, wbase, voff, doff, b0 + 2 * U, nb, bstride);
        acc = accumulate_batch<U>(b, xs, xd, L, b0 + U, nb, acc);
    }
    acc = acc + xor_f(acc, 4);
    acc = acc + xor_f(acc, 2);
    acc = acc + xor_f(acc, 1);
    if (L == 0 && row < m_weight) {
        if (__builtin_isnan(acc) || xm128)
            acc = t_order_cell(W + (int64_t)row * wrow, bstride, LAYOUT == 0 ? 2 : 4, Xq + (int64_t)tok * bpr, nb,
                               row, tok, m_weight, (int)gridDim.y);
        out[(int64_t)tok * m_weight + row] = acc;
    }
}

// ----------------------------------------------------------------------------
// The same order T with the memory latency taken off the chains: a workgroup
// holds 8 weight rows of one token and has 5 waves.  Waves 1-4 (producers)
// compute the block products RN(RN(Ad*Bd) * float(p_L)) of 32-block chunks,
// one lane per (row, block) of a chunk, all 8 partials L of it from the block's
// 34 bytes (8 dword loads and one 16-bit load, re-aligned with v_alignbit for
// even blocks of the 34-byte layout), with the loads of the next 8 chunks in
// flight in registers, and write them to a two-slot LDS array; wave 0
// (consumer) lane (row, L) runs the reference's accumulator chain
// acc_L = prod + acc_L over the products in block order, and combines the 8
// lanes of a row as k_q8_0_gemv_T does.  The chain lanes only add, so the
// kernel streams the weights at the rate the producers keep in flight instead
// of one load latency per block.  One barrier per chunk.
// ----------------------------------------------------------------------------
constexpr int kTpChunk = 32;          // blocks per chunk
constexpr int kTpLd = kTpChunk + 4;   // product row pitch (floats), float4-aligned
constexpr int kTpAhead = 8;           // chunks in flight per producer lane

struct TpLoad {
    uint32_t w[8];  // LAYOUT 1 and odd blocks: quant dwords; even blocks: raw dwords from the block start
    uint32_t e;     // the 16-bit word w leaves out: the scale, or (even blocks) quant bytes 30-31 of L = 7
};

struct TpLane {
    const uint8_t* rowbase;  // this producer lane's weight row, block 0
    int64_t bstride;         // bytes from block b to block b+1 of the row
    int j, row8, nb;         // block within a chunk, row within the workgroup * 8
};

template <int LAYOUT>
__device__ __forceinline__ void tp_load(TpLoad& t, const TpLane& p, int c) {
    const int b = min(c * kTpChunk + p.j, p.nb - 1);
    const uint8_t* blk = p.rowbase + (int64_t)b * p.bstride;
    if (LAYOUT == 1 || (b & 1)) {
        // quant dword L at byte 2+4L (34-byte blocks, odd b: 4-byte aligned) or 4+4L (padded)
        const uint8_t* qp = blk + (LAYOUT == 0 ? 2 : 4);
#pragma unroll
        for (int k = 0; k < 8; k++) t.w[k] = ld_u32(qp + 4 * k);
        t.e = ld_u16(blk);
    } else {
        // even b of the 34-byte layout: dwords at the (aligned) block start, then bytes 32-33
#pragma unroll
        for (int k = 0; k < 8; k++) t.w[k] = ld_u32(blk + 4 * k);
        t.e = ld_u16(blk + 32);
    }
}

template <int LAYOUT>
__device__ __forceinline__ void tp_products(const TpLoad& t, const TpLane& p, float* __restrict__ prod,
                                            const uint32_t* __restrict__ xs, const float* __restrict__ xd, int c) {
    const int b = c * kTpChunk + p.j;
    if (b >= p.nb) return;
    const bool aligned = LAYOUT == 1 || (b & 1);
    const uint32_t dbits = aligned ? t.e : (t.w[0] & 0xFFFFu);
    const float scale = f16_ieee(dbits) * xd[b];
#pragma unroll
    for (int L = 0; L < 8; L++) {
        uint32_t q;
        if (aligned)
            q = t.w[L];
        else
            q = __builtin_amdgcn_alignbit(L < 7 ? t.w[L + 1] : t.e, t.w[L], 16);
        const int s = sdot4(q, xs[b * 8 + L], 0);
        prod[(p.row8 + L) * kTpLd + p.j] = scale * (float)s;
    }
}

// Step c = c0 + U: producers turn chunk c+1 (register slot (U+1)%8) into
// products and refill that slot with chunk c+9; the consumer adds chunk c.
// U is a template argument so that the register slots are indexed by constants.
template <int U, int LAYOUT>
__device__ __forceinline__ void tp_step(TpLoad (&regs)[kTpAhead], const TpLane& p, bool producer,
                                        float (*prod)[64 * kTpLd], const uint32_t* __restrict__ xs,
                                        const float* __restrict__ xd, int c0, int nch, float& acc) {
    constexpr int S = (U + 1) % kTpAhead;
    const int c = c0 + U;
    if (producer && c + 1 < nch) {
        tp_products<LAYOUT>(regs[S], p, prod[(c + 1) & 1], xs, xd, c + 1);
        if (c + 1 + kTpAhead < nch) tp_load<LAYOUT>(regs[S], p, c + 1 + kTpAhead);
    }
    if (!producer && c < nch) {
        const float* f = prod[c & 1] + threadIdx.x * kTpLd;
        const int nblk = min(kTpChunk, p.nb - c * kTpChunk);
        if (nblk == kTpChunk) {
            float4 t[kTpChunk / 4];
#pragma unroll
            for (int i = 0; i < kTpChunk / 4; i++) t[i] = reinterpret_cast<const float4*>(f)[i];
#pragma unroll
            for (int i = 0; i < kTpChunk / 4; i++) {
                acc = t[i].x + acc;
                acc = t[i].y + acc;
                acc = t[i].z + acc;
                acc = t[i].w + acc;
            }
        } else {
            for (int j = 0; j < nblk; j++) acc = f[j] + acc;
        }
    }
    __syncthreads();
}

template <int LAYOUT>
__global__ __launch_bounds__(320) void k_q8_0_gemv_TP(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Xq,
                                                       float* __restrict__ out, int m_weight, int nb) {
    extern __shared__ uint32_t lds[];
    uint32_t* xs = lds;                                   // [nb][8] activation quants
    float* xd = reinterpret_cast<float*>(lds + nb * 8);   // [nb] activation scales
    __shared__ __align__(16) float prod[2][64 * kTpLd];
    const int tid = threadIdx.x, tok = blockIdx.y, row0 = blockIdx.x * 8;
    const bool producer = tid >= 64;
    const int pp = producer ? tid - 64 : 0;
    TpLane p;
    p.j = pp & 31;
    p.row8 = (pp >> 5) * 8;
    p.nb = nb;
    const int row = min(row0 + (pp >> 5), m_weight - 1);  // rows past the end reuse the last row (outputs discarded)
    p.rowbase = W + (int64_t)row * (LAYOUT == 0 ? (int64_t)nb * kQ80Bytes : 64);
    p.bstride = LAYOUT == 0 ? kQ80Bytes : (int64_t)m_weight * 64;
    const int nch = (nb + kTpChunk - 1) / kTpChunk;
    // loads return in order, so: chunk 0, then the activation row (the first
    // barrier waits for it), then the rest of the prefetch
    // the activation row first (an L2 hit for every workgroup but the first few),
    // then the weight prefetch: loads return in order, so staging issued after
    // the prefetch would wait for all of it
    __shared__ uint32_t wave_m128[5];
    note_m128(wave_m128, stage_x<320>(xs, xd, Xq + (int64_t)tok * nb * kQ80Bytes, nb));
    TpLoad regs[kTpAhead];
    if (producer) {
#pragma unroll
        for (int c = 0; c < kTpAhead; c++)
            if (c < nch) tp_load<LAYOUT>(regs[c], p, c);
    }
    __syncthreads();
    const bool xm128 = __builtin_amdgcn_readfirstlane((int)row_m128(wave_m128, 5)) != 0;
    if (producer) {
        tp_products<LAYOUT>(regs[0], p, prod[0], xs, xd, 0);
        if (kTpAhead < nch) tp_load<LAYOUT>(regs[0], p, kTpAhead);
    }
    __syncthreads();
    float acc = 0.0f;
    static_assert(kTpAhead == 8, "one tp_step per register slot");
    for (int c0 = 0; c0 < nch; c0 += kTpAhead) {
        tp_step<0, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<1, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<2, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<3, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<4, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<5, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<6, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
        tp_step<7, LAYOUT>(regs, p, producer, prod, xs, xd, c0, nch, acc);
    }
    if (!producer) {
        acc = acc + xor_f(acc, 4);
        acc = acc + xor_f(acc, 2);
        acc = acc + xor_f(acc, 1);
        const int orow = row0 + (tid >> 3);
        if ((tid & 7) == 0 && orow < m_weight) {
            if (__builtin_isnan(acc) || xm128)
                acc = t_order_cell(W + (int64_t)orow * (LAYOUT == 0 ? (int64_t)nb * kQ80Bytes : 64), p.bstride,
                                   LAYOUT == 0 ? 2 : 4, Xq + (int64_t)tok * nb * kQ80Bytes, nb, orow, tok, m_weight,
                                   (int)gridDim.y);
            out[(int64_t)tok * m_weight + orow] = acc;
        }
    }
}

// ----------------------------------------------------------------------------
// The same order T for 34-byte rows read as 16-byte lanes, one wave per 2 rows
// and four lanes per chain, with nothing shared between the waves but the
// activation row.  The loads of k_q8_0_gemv_T (a dword and a 16-bit word per
// lane and block) reach 3.6 TB/s at the cfg2 shapes even without arithmetic;
// 16-byte lanes over the same bytes reach 5.9, and more so with 2 rows per wave
// than with 4 (4096x14336 read alone: 10.7 us against 12.5).
// Each wave streams its 2 rows in chunks of 32 blocks (1088 bytes of a row, 68
// aligned 16-byte pieces, 136 pieces for the 2 rows: 3 loads per lane, the 3rd
// on lanes 0..7) with 2 chunks in flight in registers, and stages the current
// chunk in a private LDS slot (1248-byte row pitch).  It then forms the chunk's
// 2 x 32 scale products RN(Ad*Bd) once (one per lane).
// Lane (row, L, q), lane index 32 row + 4L + q, computes the products
// RN(RN(Ad*Bd) * float(p_L)) of the blocks b with b % 4 == q: the quant dword at
// byte 34b + 2 + 4L (two aligned LDS dwords and v_alignbit), the activation
// dwords and scale products four blocks at a time from copies split by b % 4.
// The four lanes of a quad then extend the same chain
//   acc_L = RN(p_L(b) + acc_L), ..., acc_L = RN(p_L(b+3) + acc_L)
// taking block b+j's product from lane 4L+j (DPP quad_perm broadcast in the
// adds), so they hold identical accumulators.
// A wave waits only for its own loads and its own LDS writes (the LDS queue is
// in order per wave): the one workgroup barrier is the one after the
// activation row is staged.  The products, their order and the final combine
// are k_q8_0_gemv_T's, so the bits are too.  Needs nb % 32 == 0 and W 16-byte
// aligned.
//
// Every chunk step issues its 3 loads (past the last chunk a 16-byte read of the
// wave's first row that every lane shares, discarded), in a loop of whole chunk
// pairs plus an odd tail step: with no load under a branch the compiler's wait
// before a chunk's LDS writes leaves the next chunk in flight (vmcnt(3)-(5));
// with the last loads skipped by a branch it waited for every load of the wave
// once per two chunks (4096x14336: 14.0 -> 13.4 us, 2048x14336: 10.9 -> 9.4).
// ----------------------------------------------------------------------------
typedef uint32_t v_u32x4 __attribute__((ext_vector_type(4)));  // native vectors: stay in VGPRs
typedef float v_f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVChunk = 32;                  // blocks per chunk
constexpr int kVRowB = kVChunk * kQ80Bytes;  // 1088 bytes of a row per chunk
constexpr int kVPieces = kVRowB / 16;        // 68 aligned 16-byte pieces
constexpr int kVRows = 2;                    // rows per wave
constexpr int kVPitch = 1248;                // LDS row pitch, bytes
constexpr int kVWavePieces = kVRows * kVPieces;  // 136 pieces per wave and chunk
constexpr int kVPer = (kVWavePieces + 63) / 64;  // loads per lane and chunk
constexpr int kVScP = kVChunk / 4 + 4;       // (row, b%4) pitch of the scale products, floats
constexpr int kVSlot = kVRows * kVPitch + 4 * kVRows * kVScP * 4;  // LDS bytes per wave
constexpr int kVAhead = 2;                   // chunks in flight per wave
static_assert(kVPer == 3 && kVSlot % 16 == 0, "slot geometry");

// activation quant dwords: [L][b%4][nb/4 + 4] (the 32 rows of a read 4 banks apart)
__host__ __device__ constexpr int v_xpitch(int nb) { return nb / 4 + 4; }
__host__ __device__ constexpr size_t v_lds_bytes(int nb, int nw) {
    return (size_t)(32 * v_xpitch(nb) + nb) * 4 + (size_t)nw * kVSlot;
}

// the wave's own LDS writes complete before its later reads (and the compiler
// keeps them in that order)
__device__ __forceinline__ void v_lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ bool v_piece(int lane, int k) { return k < kVPer - 1 || lane + 64 * k < kVWavePieces; }

// Non-temporal: each weight byte is read once, and every 16-byte piece of a
// 128-byte line is loaded by the same instruction.  Lanes past the wave's 136
// pieces load piece 135 (off[] is clamped), an address another lane of the same
// instruction loads.  real == false: the shared 16-byte read of a step past the
// last chunk.
__device__ __forceinline__ void v_load(v_u32x4 (&v)[kVPer], const uint8_t* __restrict__ wbase,
                                       const uint32_t (&off)[kVPer], int c, bool real) {
    const uint8_t* src = wbase + (real ? (uint32_t)c * kVRowB : 0u);
#pragma unroll
    for (int k = 0; k < kVPer; k++)
        v[k] = __builtin_nontemporal_load(reinterpret_cast<const v_u32x4*>(src + (real ? off[k] : 0u)));
}

// v read from lane (lane & ~3) + SEL of each quad
template <int SEL>
__device__ __forceinline__ float v_quad(float v) {
    constexpr int ctrl = SEL | (SEL << 2) | (SEL << 4) | (SEL << 6);  // quad_perm
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, true));
}

// Chunk c = c0 + U < nch (register slot U holds it; U is a template argument so
// that the slots are indexed by constants): stage it, refill slot U with chunk
// c + kVAhead, scale products, chains.
template <int U>
__device__ __forceinline__ void v_step(v_u32x4 (&pf)[kVAhead][kVPer], uint8_t* slot, float* sc,
                                       const uint8_t* __restrict__ wbase, const uint32_t (&off)[kVPer],
                                       const uint32_t (&dst)[kVPer], int lane, int c0, int nch,
                                       const uint32_t* __restrict__ xs, const float* __restrict__ xd, int xp,
                                       float& acc) {
    const int c = c0 + U;
#pragma unroll
    for (int k = 0; k < kVPer; k++)
        if (v_piece(lane, k)) *reinterpret_cast<v_u32x4*>(slot + dst[k]) = pf[U][k];
    v_load(pf[U], wbase, off, c + kVAhead, c + kVAhead < nch);
    v_lds_order();
    {
        const int r = lane / kVChunk, bb = lane % kVChunk;  // kVRows * kVChunk == 64
        const uint32_t ad = *reinterpret_cast<const uint16_t*>(slot + r * kVPitch + bb * kQ80Bytes);
        sc[(4 * r + (bb & 3)) * kVScP + (bb >> 2)] = f16_ieee(ad) * xd[c * kVChunk + bb];
    }
    v_lds_order();
    const int q = lane & 3, L = (lane >> 2) & 7, rr = lane >> 5;
    const uint8_t* rowp = slot + rr * kVPitch;
    const uint32_t* xl = xs + (4 * L + q) * xp + c * (kVChunk / 4);
    const float* sr = sc + (4 * rr + q) * kVScP;
    // this lane's quant dword in block bb + q (bb % 4 == 0) is at 34 bb + ob; 34 bb = 0 mod 4
    const int ob = 34 * q + 2 + 4 * L, oa = ob & ~3, sh = (ob & 3) * 8;
#pragma unroll
    for (int b16 = 0; b16 < kVChunk; b16 += 16) {
        const v_u32x4 xq = *reinterpret_cast<const v_u32x4*>(xl + b16 / 4);  // blocks b16+q, b16+4+q, ...
        const v_f32x4 s4 = *reinterpret_cast<const v_f32x4*>(sr + b16 / 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int bb = b16 + 4 * j;
            const uint32_t lo = *reinterpret_cast<const uint32_t*>(rowp + 34 * bb + oa);
            const uint32_t hi = *reinterpret_cast<const uint32_t*>(rowp + 34 * bb + oa + 4);
            const int p = sdot4(__builtin_amdgcn_alignbit(hi, lo, sh), xq[j], 0);
            const float mine = s4[j] * (float)p;
            acc = v_quad<0>(mine) + acc;  // block bb
            acc = v_quad<1>(mine) + acc;  // block bb + 1
            acc = v_quad<2>(mine) + acc;  // block bb + 2
            acc = v_quad<3>(mine) + acc;  // block bb + 3
        }
    }
}

// NW waves of 2 rows per workgroup; x quants in XR dwords per thread (nb*8 <= XR*64*NW).
// XR = 4 (K <= 4096): at most 72 VGPRs, 7 waves per SIMD, which the 7,168 waves
// of 14336x4096 need to be resident at once (84 VGPRs unbounded: 13.5 -> 12.8 us;
// the larger XR spill under that bound and are left unbounded).
template <int NW, int XR>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(XR <= 4 ? 7 : 1)))
void k_q8_0_gemv_V(const uint8_t* __restrict__ W,
                                                        const uint8_t* __restrict__ Xq, float* __restrict__ out,
                                                        int m_weight, int nb) {
    static_assert(kVAhead == 2, "one v_step call per chunk in flight");
    static_assert(kVRows * kVChunk == 64, "one scale product per lane");
    constexpr int NT = 64 * NW;
    extern __shared__ __align__(16) uint32_t lds[];
    const int xp = v_xpitch(nb);
    uint32_t* xs = lds;                                          // quant dword L of block b at (4L + b%4)*xp + b/4
    float* xd = reinterpret_cast<float*>(lds + 32 * xp);         // [nb] activation scales
    const int tid = threadIdx.x, lane = tid & 63, tok = blockIdx.y;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t* slot = reinterpret_cast<uint8_t*>(lds + 32 * xp + nb) + wave * kVSlot;
    float* sc = reinterpret_cast<float*>(slot + kVRows * kVPitch);  // [row][b%4][kVScP]
    const int row0 = (blockIdx.x * NW + wave) * kVRows, nch = nb / kVChunk;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    // rows past m_weight re-read row m_weight-1 (their cells are not written)
    const int row0c = min(row0, m_weight - 1);
    const uint8_t* wbase = W + (int64_t)row0c * bpr;
    // the activation row into registers first (loads return in order)
    const uint8_t* xr = Xq + (int64_t)tok * bpr;
    constexpr int XD = (XR + 7) / 8;  // nb <= XD * NT scales
    uint32_t xq[XR], xh[XD];
#pragma unroll
    for (int u = 0; u < XR; u++) {
        const int i = min(tid + u * NT, nb * 8 - 1);
        xq[u] = ld_u32(xr + (int64_t)(i >> 3) * kQ80Bytes + 2 + 4 * (i & 7));
    }
#pragma unroll
    for (int u = 0; u < XD; u++) xh[u] = ld_u16(xr + (int64_t)min(tid + u * NT, nb - 1) * kQ80Bytes);
    // piece k of this lane: f = min(lane + 64k, 135) is row f/68, piece f%68 of the chunk
    uint32_t off[kVPer], dst[kVPer];
#pragma unroll
    for (int k = 0; k < kVPer; k++) {
        const int f = min(lane + 64 * k, kVWavePieces - 1), r = f / kVPieces, p = f % kVPieces;
        off[k] = (uint32_t)((min(row0 + r, m_weight - 1) - row0c) * bpr) + 16u * p;
        dst[k] = (uint32_t)(r * kVPitch + 16 * p);
    }
    v_u32x4 pf[kVAhead][kVPer];
#pragma unroll
    for (int a = 0; a < kVAhead; a++)
        if (a < nch) v_load(pf[a], wbase, off, a, true);
    uint32_t any_m128 = 0;
#pragma unroll
    for (int u = 0; u < XR; u++) {
        const int i = tid + u * NT, b = i >> 3;
        if (i < nb * 8) {
            xs[(4 * (i & 7) + (b & 3)) * xp + (b >> 2)] = xq[u];
            any_m128 |= has_m128(xq[u]);
        }
    }
    __shared__ uint32_t wave_m128[NW];
    note_m128(wave_m128, any_m128);
#pragma unroll
    for (int u = 0; u < XD; u++)
        if (tid + u * NT < nb) xd[tid + u * NT] = f16_ieee(xh[u]);
    __syncthreads();
    // read once here, off the kernel's tail; wave-uniform
    const bool xm128 = __builtin_amdgcn_readfirstlane((int)row_m128(wave_m128, NW)) != 0;
    float acc = 0.0f;
    // whole pairs of chunks, then an odd last one: no step of the loop body can be
    // skipped, so every trip issues the same loads in the same order
    int c0 = 0;
    for (; c0 + 1 < nch; c0 += kVAhead) {
        v_step<0>(pf, slot, sc, wbase, off, dst, lane, c0, nch, xs, xd, xp, acc);
        v_step<1>(pf, slot, sc, wbase, off, dst, lane, c0, nch, xs, xd, xp, acc);
    }
    if (c0 < nch) v_step<0>(pf, slot, sc, wbase, off, dst, lane, c0, nch, xs, xd, xp, acc);
    // lanes 4L..4L+3 hold the same acc_L (L at lane bits 2-4): k_q8_0_gemv_T's combine over L
    acc = acc + xor_f(acc, 16);
    acc = acc + xor_f(acc, 8);
    acc = acc + xor_f(acc, 4);
    const int row = row0 + (lane >> 5);
    if ((lane & 31) == 0 && row < m_weight) {
        if (__builtin_isnan(acc) || xm128)
            acc = t_order_cell(W + (int64_t)row * bpr, kQ80Bytes, 2, xr, nb, row, tok, m_weight, (int)gridDim.y);
        out[(int64_t)tok * m_weight + row] = acc;
    }
}

// Plain form of the same order for activation rows too long to stage in LDS.
template <int LAYOUT = 0>
__global__ __launch_bounds__(256) void k_q8_0_gemm_T(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Xq,
                                                     float* __restrict__ out, int m_weight, int nb) {
    const int lane = threadIdx.x & 63;
    const int L = lane & 7;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
    const int tok = blockIdx.y;
    if ((row & ~7) >= m_weight) return;
    const int rr = min(row, m_weight - 1);
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const uint8_t* wr = W + (int64_t)rr * (LAYOUT == 0 ? bpr : 64);
    const uint8_t* xr = Xq + (int64_t)tok * bpr;
    float acc = 0.0f;
    uint32_t any_m128 = 0;  // the cell's 8 lanes see every activation quant
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = wr + (int64_t)b * (LAYOUT == 0 ? (int64_t)kQ80Bytes : (int64_t)m_weight * 64);
        const uint8_t* xb = xr + (int64_t)b * kQ80Bytes;
        const uint32_t wv = ld_u32(wb + (LAYOUT == 0 ? 2 : 4) + 4 * L);
        const uint32_t xv = ld_u32(xb + 2 + 4 * L);
        any_m128 |= has_m128(xv);
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
    any_m128 |= (uint32_t)xor_i((int)any_m128, 4);
    any_m128 |= (uint32_t)xor_i((int)any_m128, 2);
    any_m128 |= (uint32_t)xor_i((int)any_m128, 1);
    if (L == 0 && row < m_weight) {
        if (__builtin_isnan(acc) || any_m128 != 0)
            acc = t_order_cell(W + (int64_t)row * (LAYOUT == 0 ? bpr : 64),
                               LAYOUT == 0 ? (int64_t)kQ80Bytes : (int64_t)m_weight * 64, LAYOUT == 0 ? 2 : 4,
                               Xq + (int64_t)tok * bpr, nb, row, tok, m_weight, (int)gridDim.y);
        out[(int64_t)tok * m_weight + row] = acc;
    }
}

// Every cell of an empty (K = 0) product is the empty sum, +0.0.
__global__ __launch_bounds__(256) void k_fill_zero(float* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = 0.0f;
}

void launch_fill_zero(float* out, int64_t n, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n);
}

// k_q8_0_gemv_V with NW waves per workgroup for nb blocks, or NULL when the
// activation row does not fit XR <= 32 dwords per thread.
template <int NW>
static const void* v_kernel(int nb) {
    constexpr int NT = 64 * NW;
    if (nb * 8 <= 4 * NT) return reinterpret_cast<const void*>(&k_q8_0_gemv_V<NW, 4>);
    if (nb * 8 <= 8 * NT) return reinterpret_cast<const void*>(&k_q8_0_gemv_V<NW, 8>);
    if (nb * 8 <= 16 * NT) return reinterpret_cast<const void*>(&k_q8_0_gemv_V<NW, 16>);
    if (nb * 8 <= 32 * NT) return reinterpret_cast<const void*>(&k_q8_0_gemv_V<NW, 32>);
    return nullptr;
}

// The wide-load kernel where it is measured faster (MI355X, weights beyond the
// MALL), by 2-row waves w = ceil(m_weight/2) * m_tokens: from w >= 256, 4 waves
// per workgroup (8 when the activation row needs them: nb > 1024).  Against the
// 4-row form it replaces (probe copies, eager, one box): 14336x4096 12.8 us
// (13.6), 4096x14336 13.4 (15.2), 2048x14336 9.4 (13.4), 6144x4096 7.1 (8.5),
// 4096x4096 5.9 (6.9), 1024x4096 4.5 (5.6), 512x4096 4.4 (5.5), 28672x4096 22.9
// (23.1).  Returns false when the shape or W's alignment does not fit.
static bool launch_wide(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int nb,
                        hipStream_t s) {
    if (nb % kVChunk != 0 || (reinterpret_cast<uintptr_t>(Wq) & 15) != 0) return false;
    const int64_t waves = (int64_t)((m_weight + kVRows - 1) / kVRows) * m_tokens;
    if (waves < 256) return false;
    int nw = 4;
    const void* f = v_kernel<4>(nb);
    if (f == nullptr) {  // a long activation row: 8 waves stage it
        nw = 8;
        f = v_kernel<8>(nb);
    }
    const size_t lds = v_lds_bytes(nb, nw);
    if (f == nullptr || lds > 160 * 1024) return false;
    if (lds > 64 * 1024) {
        // more than 64 KB of dynamic LDS is asked for once per process (only the
        // 8-wave, 32-register form can need it)
        static std::once_flag once;
        static bool lds_ok = false;
        std::call_once(once, [] {
            lds_ok = hipFuncSetAttribute(v_kernel<8>(2048), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) ==
                     hipSuccess;
            (void)hipGetLastError();
        });
        if (!lds_ok) return false;
    }
    const int rows = kVRows * nw;
    void* args[] = {const_cast<uint8_t**>(&Wq), const_cast<uint8_t**>(&Xq), &out, &m_weight, &nb};
    (void)hipLaunchKernel(f, dim3((m_weight + rows - 1) / rows, m_tokens), dim3(64 * nw), args, lds, s);
    return true;
}

template <int LAYOUT>
static void dispatch_T(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                       hipStream_t s) {
    const int nb = K / 32;
    if (nb == 0) {  // the kernels below index block nb-1
        launch_fill_zero(out, (int64_t)m_weight * m_tokens, s);
        return;
    }
    if (LAYOUT == 0 && launch_wide(Wq, Xq, out, m_weight, m_tokens, nb, s)) return;
    const int waves = (m_weight + 7) / 8;
    const size_t lds = (size_t)nb * 36;
    if (lds > 64 * 1024) {
        hipLaunchKernelGGL(k_q8_0_gemm_T<LAYOUT>, dim3((waves + 3) / 4, m_tokens), dim3(256), 0, s, Wq, Xq, out,
                           m_weight, nb);
        return;
    }
    // shapes measured on MI355X (graph, weights beyond the MALL): with many waves
    // the pipelined kernel with 16-block batches and 4 waves per workgroup
    // (14336x4096: 20.1 us vs 32.0 for the producer/consumer kernel); with fewer
    // waves the producer/consumer kernel (4096x14336: 24.2 us vs 38.4 for 32-block
    // batches; 4096x4096: 9.2 vs 13.0; 1024x4096: 6.7 vs 12.5)
    if (waves * m_tokens >= 1024)
        hipLaunchKernelGGL((k_q8_0_gemv_T<16, 4, LAYOUT>), dim3((waves + 3) / 4, m_tokens), dim3(256), lds, s, Wq, Xq,
                           out, m_weight, nb);
    else if (lds + sizeof(float) * 2 * 64 * kTpLd <= 64 * 1024)
        hipLaunchKernelGGL((k_q8_0_gemv_TP<LAYOUT>), dim3((m_weight + 7) / 8, m_tokens), dim3(320), lds, s, Wq, Xq, out,
                           m_weight, nb);
    else
        hipLaunchKernelGGL((k_q8_0_gemv_T<32, 2, LAYOUT>), dim3((waves + 1) / 2, m_tokens), dim3(128), lds, s, Wq,
                           Xq, out, m_weight, nb);
}

void launch_q8_0_dispatch_T(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                            hipStream_t s) {
    dispatch_T<0>(Wq, Xq, out, m_weight, m_tokens, K, s);
}

void launch_q8_pad64_dispatch_T(const uint8_t* Wp, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                                hipStream_t s) {
    dispatch_T<1>(Wp, Xq, out, m_weight, m_tokens, K, s);
}

// ----------------------------------------------------------------------------
// fp32 [N, K] -> the padded Q8 layout of inference/llamatov_c_inference.py:88-100:
// per (row n, block b) of 32 values, d = RN(max(amax, 1e-10) / 127) (float32),
// q = clip(round-half-even(RN(x / d)), -128, 127), record (b, n) at byte
// (b*N + n)*64 = {f16(d) RNE, 0, 0, q[32], 28 zero bytes}.  32 lanes per record
// (lane = element), so the reads of consecutive records are contiguous.
// As numpy computes it: a NaN in the block carries through max, clip and /127
// into d (float16 0x7E00) and every quant is 0 (NaN cast to int8); with an Inf
// (d = Inf) Inf/Inf is NaN and its quant 0.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q8_pad64(const float* __restrict__ x, uint8_t* __restrict__ out, int N,
                                                  int nb) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rec = g >> 5;  // n * nb + b: the 32 lanes of a record stay together
    const int e = (int)(g & 31);
    if (rec >= (int64_t)N * nb) return;
    const int64_t n = rec / nb, b = rec - n * nb;
    const float v = x[rec * 32 + e];
    float amax = fabsf(v);
#pragma unroll
    for (int mask = 1; mask < 32; mask <<= 1) amax = fmaxf(amax, xor_f(amax, mask));
    // a NaN anywhere in the record (its 32 lanes are one half of the wave)
    const bool nan_rec = ((uint64_t)__ballot(__builtin_isnan(v)) >> (threadIdx.x & 32) & 0xFFFFFFFFull) != 0;
    amax = fmaxf(amax, 1e-10f);
    const float d = amax / 127.0f;
    const float r = __builtin_rintf(v / d);
    const float qf = (nan_rec || __builtin_isnan(r)) ? 0.0f : fminf(fmaxf(r, -128.0f), 127.0f);
    uint8_t* o = out + (b * N + n) * 64;
    o[4 + e] = (uint8_t)(int8_t)(int)qf;
    if (e < 28) o[36 + e] = 0;
    if (e == 0) {
        const uint16_t h = nan_rec ? (uint16_t)0x7E00 : __builtin_bit_cast(uint16_t, (_Float16)d);
        *reinterpret_cast<uint32_t*>(o) = (uint32_t)h;
    }
}

void launch_q8_pad64(const float* x, uint8_t* out, int N, int K, hipStream_t s) {
    const int64_t threads = (int64_t)N * (K / 32) * 32;
    if (threads == 0) return;
    hipLaunchKernelGGL(k_q8_pad64, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, out, N, K / 32);
}

}  // namespace bpdq

namespace bpdq {

// ----------------------------------------------------------------------------
// Prefill GEMM in the scalar order S (bench/bpd_gemm_q8_0_cpu.c:102-131,
// bench/bpd_cpu.c:4263-4280): per output cell
//   acc = +0.0;  for b in blocks: acc = RN(acc + RN(float(S_b) * RN(Ad_b * Bd_b)))
// with S_b the exact int32 dot of the cell's two 32-element blocks.  One K step
// of v_mfma_i32_32x32x32_i8 covers exactly one Q8_0 block, so with a zero
// accumulator it yields S_b for a 32 x 32 tile of cells; the fp32 epilogue then
// applies the block's scale in order.  Bit-identical to the scalar (-O2) build
// of bpd_qmatmul_q8_0_dispatch_cpu / bpd_qmatmul_q8_0_llamafile_cpu.
//
// Workgroup: 4 waves in 2 x 2, tile 128 weight rows x 128 tokens; each wave
// 64 x 64 = 2 x 2 MFMA tiles.  Blocks are staged KB at a time through LDS
// (double buffered), quants 32-byte aligned per (row, block), scales as fp32.
// A lane feeds row (lane % 32) of A and column (lane % 32) of B with the same
// 16-byte half of the block (lane / 32), so every K index of A meets the same K
// index of B.  Output lane layout of a 32x32 tile: register r of lane l holds
// row 8(r/4) + 4(l/32) + r%4, column l%32.
// ----------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

// ----------------------------------------------------------------------------
// NaN cells of the scalar order S.  The reference computes
//   acc = acc + float(S_b) * (Ad*Bd)   over blocks b in order
// on x86, where the first NaN of the chain sticks (acc + p keeps acc's NaN), a
// NaN factor comes out quieted (the first operand's when both are NaN) and
// Inf*0, Inf-Inf give the default NaN.  Two reference forms differ in their NaN
// bits:
//   kSNanTile (the scalar tiles, bench/bpd_gemm_q8_0_cpu.c:112-128): scales by
//     the ldexpf decode of :13-26 (an f16 NaN becomes +/-0x7FC00000, no payload);
//     the build puts Bd first in Ad*Bd;
//   kSNanQdot (bpd_qdot_q8_0_q8_0_cpu's scalar form, bench/bpd_cpu.c:4263-4280,
//     which the scalar build's llamafile entry uses): the magic-number decode
//     (payload kept); the weight scale first.
// A finite scale product keeps a finite accumulator finite (|S_b*Ad*Bd| < 2^51)
// and an infinite one unchanged, so only blocks with an Inf or NaN scale can
// change the state, and the first NaN event fixes the bits.  Called only for a
// cell whose sum came out NaN; NaN-ness itself is the same on every IEEE machine.
// ----------------------------------------------------------------------------
constexpr int kSNanTile = 0;
constexpr int kSNanQdot = 1;
static_assert(kSNanTile != kSNanQdot, "the two NaN forms");

__device__ __forceinline__ float f16_ref(uint32_t h, int mode) {
    if (!f16_is_nan(h)) return f16_ieee(h);
    return mode == kSNanTile ? __uint_as_float(((h & 0x8000u) << 16) | 0x7FC00000u) : f16_nan_x86(h);
}

__device__ __noinline__ float s_order_nan_bits(const uint8_t* __restrict__ wrow, const uint8_t* __restrict__ xrow,
                                               int nb, int mode) {
    float acc = 0.0f;  // stands for any finite value
    for (int b = 0; b < nb; b++) {
        const uint8_t* wb = wrow + (int64_t)b * kQ80Bytes;
        const uint8_t* xb = xrow + (int64_t)b * kQ80Bytes;
        const uint32_t hw = (uint32_t)wb[0] | ((uint32_t)wb[1] << 8);
        const uint32_t hx = (uint32_t)xb[0] | ((uint32_t)xb[1] << 8);
        if (!f16_exp31(hw) && !f16_exp31(hx)) continue;
        const float fw = f16_ref(hw, mode), fx = f16_ref(hx, mode);
        const float first = mode == kSNanTile ? fx : fw, second = mode == kSNanTile ? fw : fx;
        const float delta = first * second;
        // a NaN product: p = float(S_b) * delta is delta's NaN, and acc + p is p's
        if (__builtin_isnan(delta)) return x86_nan_of(first, second);
        // delta is +/-Inf: p = +/-Inf, or the default NaN when S_b = 0
        int sumi = 0;
        for (int j = 0; j < 32; j++) sumi += (int)(int8_t)wb[2 + j] * (int)(int8_t)xb[2 + j];
        if (sumi == 0) return __uint_as_float(kX86NaN);
        const float p = sumi < 0 ? -delta : delta;
        if (__builtin_isinf(acc) && acc != p) return __uint_as_float(kX86NaN);  // Inf - Inf
        acc = p;
    }
    return acc;
}

constexpr int kGT = 128;  // tile rows = tile tokens
constexpr int kGB = 4;    // blocks per LDS stage

struct GemmLds {
    uint8_t aq[2][kGB][kGT][32];
    uint8_t bq[2][kGB][kGT][32];
    float ad[2][kGB][kGT];
    float bd[2][kGB][kGT];
};

// One (row, block) of a Q8_0 matrix: scale bits and the 32 quants.
struct BlkRegs {
    uint32_t d;
    uint32_t q[8];
};

__device__ __forceinline__ void load_blk(BlkRegs& r, const uint8_t* __restrict__ p) {
    r.d = ld_u16(p);
#pragma unroll
    for (int j = 0; j < 8; j++) r.q[j] = ld_u32(p + 2 + 4 * j);
}

// Thread t stages pairs t, t+256 of A (row-major over 128 rows x kGB blocks) and
// the same of B.
__device__ __forceinline__ void stage_load(BlkRegs (&ra)[2], BlkRegs (&rb)[2], const uint8_t* __restrict__ W,
                                           const uint8_t* __restrict__ X, int m0, int n0, int m_weight,
                                           int m_tokens, int b0, int nb, int64_t bpr) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int p = threadIdx.x + 256 * i;
        const int rr = p & (kGT - 1), u = p >> 7;
        const int blk = min(b0 + u, nb - 1);
        load_blk(ra[i], W + (int64_t)min(m0 + rr, m_weight - 1) * bpr + (int64_t)blk * kQ80Bytes);
        load_blk(rb[i], X + (int64_t)min(n0 + rr, m_tokens - 1) * bpr + (int64_t)blk * kQ80Bytes);
    }
}

__device__ __forceinline__ void stage_store(GemmLds& s, int buf, const BlkRegs (&ra)[2], const BlkRegs (&rb)[2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int p = threadIdx.x + 256 * i;
        const int rr = p & (kGT - 1), u = p >> 7;
        uint4* qa = reinterpret_cast<uint4*>(s.aq[buf][u][rr]);
        qa[0] = make_uint4(ra[i].q[0], ra[i].q[1], ra[i].q[2], ra[i].q[3]);
        qa[1] = make_uint4(ra[i].q[4], ra[i].q[5], ra[i].q[6], ra[i].q[7]);
        uint4* qb = reinterpret_cast<uint4*>(s.bq[buf][u][rr]);
        qb[0] = make_uint4(rb[i].q[0], rb[i].q[1], rb[i].q[2], rb[i].q[3]);
        qb[1] = make_uint4(rb[i].q[4], rb[i].q[5], rb[i].q[6], rb[i].q[7]);
        s.ad[buf][u][rr] = f16_ieee(ra[i].d);
        s.bd[buf][u][rr] = f16_ieee(rb[i].d);
    }
}

__global__ __launch_bounds__(256) void k_q8_0_gemm_S(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                     float* __restrict__ out, int m_weight, int m_tokens, int nb,
                                                     int nan_mode) {
    __shared__ GemmLds s;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wr = wave >> 1, wc = wave & 1;
    const int m0 = blockIdx.x * kGT, n0 = blockIdx.y * kGT;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const int col = lane & 31, half = lane >> 5;

    float acc[2][2][16];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[rt][ct][r] = 0.0f;

    BlkRegs ra[2], rb[2];
    const int nstages = (nb + kGB - 1) / kGB;
    stage_load(ra, rb, W, X, m0, n0, m_weight, m_tokens, 0, nb, bpr);
    stage_store(s, 0, ra, rb);
    __syncthreads();

    for (int st = 0; st < nstages; st++) {
        const int buf = st & 1;
        if (st + 1 < nstages) stage_load(ra, rb, W, X, m0, n0, m_weight, m_tokens, (st + 1) * kGB, nb, bpr);
        for (int u = 0; u < kGB; u++) {
            if (st * kGB + u >= nb) break;
            i32x4 fa[2], fb[2];
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
                fa[rt] = *reinterpret_cast<const i32x4*>(&s.aq[buf][u][wr * 64 + rt * 32 + col][16 * half]);
#pragma unroll
            for (int ct = 0; ct < 2; ct++)
                fb[ct] = *reinterpret_cast<const i32x4*>(&s.bq[buf][u][wc * 64 + ct * 32 + col][16 * half]);
            // scale products RN(Ad*Bd) of every cell as a rank-1 fp32 MFMA: lanes 0-31
            // give K index 0 (row / column scale), lanes 32-63 K index 1 (zero), so
            // D = Ad*Bd + 0*0 + 0, rounded once.  |Ad*Bd| >= 2^-48 or 0 (f16 inputs),
            // never an fp32 subnormal.
            float av[2], bv[2];
#pragma unroll
            for (int rt = 0; rt < 2; rt++) av[rt] = half ? 0.0f : s.ad[buf][u][wr * 64 + rt * 32 + col];
#pragma unroll
            for (int ct = 0; ct < 2; ct++) bv[ct] = half ? 0.0f : s.bd[buf][u][wc * 64 + ct * 32 + col];
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    const i32x16 zero = {0};
                    const f32x16 fzero = {0.0f};
                    const i32x16 sb = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[rt], fb[ct], zero, 0, 0, 0);
                    const f32x16 delta = __builtin_amdgcn_mfma_f32_32x32x2f32(av[rt], bv[ct], fzero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float prod = (float)sb[r] * delta[r];
                        acc[rt][ct][r] = acc[rt][ct][r] + prod;
                    }
                }
            }
        }
        if (st + 1 < nstages) {
            __syncthreads();  // everyone is done reading the buffer about to be overwritten
            stage_store(s, buf ^ 1, ra, rb);
        }
        __syncthreads();
    }

#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            const int tok = n0 + wc * 64 + ct * 32 + col;
            if (tok >= m_tokens) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wr * 64 + rt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (row >= m_weight) continue;
                float v = acc[rt][ct][r];
                if (__builtin_isnan(v)) v = s_order_nan_bits(W + row * bpr, X + tok * bpr, nb, nan_mode);
                out[(int64_t)tok * m_weight + row] = v;
            }
        }
}

// ----------------------------------------------------------------------------
// The same GEMM when K is a multiple of 128 and W, X are 4-byte aligned, with
// coalesced staging and more waves.  A workgroup owns 32*RT weight rows x 128
// tokens; its 2*RT waves each own 32 rows x 64 tokens (two 32x32 MFMA tiles).
// A half-stage is 4 blocks: the bytes of one row are 136 contiguous bytes, and
// thread pair (2r, 2r+1) stages them for row r of W (first 32*RT rows) or of X
// (next 128): thread p of the pair takes blocks 2p, 2p+1 = 68 contiguous bytes
// in 17 dword loads.  In registers block 2p's scale is the low half of dword 0
// and its quants start 2 bytes into dword 0 (one v_alignbit per dword); block
// 2p+1's scale is the high half of dword 8, its quants dwords 9..16.  Two LDS
// slots alternate: while one is computed, the next half-stage is loaded and
// written to the other, one barrier per half-stage.  Many waves per CU let the
// MFMA latency of one wave hide behind the fp32 epilogue of others.  The scales
// are kept as f16 bits and read straight into the scale MFMA's operand, lanes
// 32-63 from a zero row; the quants are swizzled (h_swz) so that the LDS
// accesses are free of bank conflicts (measured: 9.6M conflict cycles per
// launch at cfg4 before, 0.46M after; 121 -> 113 us with the f16 operands).
// ----------------------------------------------------------------------------
constexpr int kGH = 4;  // blocks per half-stage

typedef unsigned int u32x4h __attribute__((ext_vector_type(4)));

// Staging thread t takes part h_part(t) (blocks 2p, 2p+1 of the half-stage) of
// staged row h_row(t): a thread pair covers a row's 136 contiguous bytes.
__device__ __forceinline__ int h_part(int t) { return t & 1; }
__device__ __forceinline__ int h_row(int t) { return t >> 1; }
// The two 16-byte halves of the 32 quants of block b, row r sit swapped when
// bit 2 of r xor bit 3 of r xor bit 1 of b is set.  The MFMA operand reads of
// 8 or 16 consecutive lanes (rows r..r+15, one half, one block) then touch
// 16-byte bank groups that are all different modulo 128 or 256 bytes, and so do
// the staging writes (rows r..r+7, blocks 2p of both parts).
__device__ __forceinline__ int h_swz(int row, int b) { return ((row >> 2) ^ (row >> 3) ^ (b >> 1)) & 1; }

template <int RT>
struct __align__(16) GemmLdsH {
    uint8_t qa[2][kGH][32 * RT][32];  // [slot][block][weight row][quants]
    uint8_t qb[2][kGH][kGT][32];      // [slot][block][token][quants]
    // f16 scale bits (high half zero); rows 32*RT and kGT are zero, for lanes 32-63
    uint32_t da[2][kGH][32 * RT + 1];
    uint32_t db[2][kGH][kGT + 1];
};

// Staging passes: 64*RT + 2*kGT staging threads (a pair per W row and per
// token) over the NT threads of the workgroup.
template <int RT, int NT>
__host__ __device__ constexpr int h_passes() { return (64 * RT + 2 * kGT + NT - 1) / NT; }

// A thread's staged words: 17 per pass.
template <int RT, int NT>
using HRaw = uint32_t[h_passes<RT, NT>()][17];

// W2 (SwiGLU pairs, else null): staged weight rows 16RT..32RT-1 are rows
// m0 .. m0 + 16RT - 1 of W2, the rows below them the same rows of W.
template <int RT, int NT>
__device__ __forceinline__ void half_load(HRaw<RT, NT>& raw, const uint8_t* __restrict__ W,
                                          const uint8_t* __restrict__ W2, const uint8_t* __restrict__ X, int m0,
                                          int n0, int m_weight, int m_tokens, int b0, int64_t bpr) {
#pragma unroll
    for (int ps = 0; ps < h_passes<RT, NT>(); ps++) {
        // threads past the last staged row repeat its loads (the store skips them)
        const int t = min((int)threadIdx.x + ps * NT, 64 * RT + 2 * kGT - 1);
        const int p = h_part(t), q = h_row(t);
        const bool wrow = q < 32 * RT;
        const int row = wrow ? q : q - 32 * RT;
        const bool second = W2 != nullptr && row >= 16 * RT;
        const uint8_t* src = wrow ? (second ? W2 : W) + (int64_t)min(m0 + (second ? row - 16 * RT : row), m_weight - 1) * bpr
                                  : X + (int64_t)min(n0 + row, m_tokens - 1) * bpr;
        src += (int64_t)(b0 + 2 * p) * kQ80Bytes;
#pragma unroll
        for (int k = 0; k < 17; k++) raw[ps][k] = *reinterpret_cast<const uint32_t*>(src + 4 * k);
    }
}

template <int RT>
__device__ __forceinline__ void half_store_one(GemmLdsH<RT>& s, int slot, const uint32_t (&d)[17], int t) {
    if (t >= 64 * RT + 2 * kGT) return;
    const int p = h_part(t), rq = h_row(t);
    const bool wrow = rq < 32 * RT;
    const int row = wrow ? rq : rq - 32 * RT;
    uint32_t q[8];
#pragma unroll
    for (int k = 0; k < 8; k++) q[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
    uint4* d0 = reinterpret_cast<uint4*>(wrow ? s.qa[slot][2 * p][row] : s.qb[slot][2 * p][row]);
    uint4* d1 = reinterpret_cast<uint4*>(wrow ? s.qa[slot][2 * p + 1][row] : s.qb[slot][2 * p + 1][row]);
    const int sw = h_swz(row, 2 * p);
    d0[sw] = make_uint4(q[0], q[1], q[2], q[3]);
    d0[sw ^ 1] = make_uint4(q[4], q[5], q[6], q[7]);
    d1[sw] = make_uint4(d[9], d[10], d[11], d[12]);
    d1[sw ^ 1] = make_uint4(d[13], d[14], d[15], d[16]);
    uint32_t* ds0 = wrow ? &s.da[slot][2 * p][row] : &s.db[slot][2 * p][row];
    uint32_t* ds1 = wrow ? &s.da[slot][2 * p + 1][row] : &s.db[slot][2 * p + 1][row];
    *ds0 = d[0] & 0xFFFFu;
    *ds1 = d[8] >> 16;
}

template <int RT, int NT>
__device__ __forceinline__ void half_store(GemmLdsH<RT>& s, int slot, const HRaw<RT, NT>& raw) {
#pragma unroll
    for (int ps = 0; ps < h_passes<RT, NT>(); ps++) half_store_one<RT>(s, slot, raw[ps], threadIdx.x + ps * NT);
}

// Up to kGemmMulti weight matrices that share the activation rows X (a prefill's
// Q, K and V) in one launch: workgroup column bx takes row block bx - first[i]
// of matrix i.
constexpr int kGemmMulti = 3;
struct GemmW {
    const uint8_t* w[kGemmMulti];
    float* out[kGemmMulti];
    int m[kGemmMulti];
    int first[kGemmMulti + 1];  // row blocks before matrix i
    uint8_t* yq;                // SwiGLU pairs: Q8_0 rows of y = silu(gate) * up, m[0] / 32 blocks per token
};

// Workgroup b of nP * nT (row panels x token tiles) takes panel bx, token tile
// by.  Workgroups go to the 8 XCDs round robin (b % 8), each with its own L2:
// when nP divides into 8, panel p runs on XCD p % 8 and its nT token tiles are
// numbered within one run of 8 nT workgroups, so they run together and read the
// panel's weight rows from one L2 (numbered panel-major, tiles of one panel ran
// a whole grid row apart, and a launch of more workgroups than fit at once read
// each panel twice).
__device__ __forceinline__ void sh_tile(int b, int nP, int nT, int& bx, int& by) {
    if ((nP & 7) == 0) {
        const int g = b / (8 * nT), r = b % (8 * nT);
        by = r >> 3;
        bx = 8 * g + (r & 7);
    } else {
        bx = b % nP;
        by = b / nP;
    }
}

// CT column tiles of 32 tokens per wave: 2 (waves of 32 rows x 64 tokens, the
// cfg4 form) or 1 (32 x 32: twice the waves for launches that leave SIMDs with
// one wave each).
// The SwiGLU epilogue: waves wr >= RT/2 hold up rows, waves wr - RT/2 the same
// gate rows (register r of lane l: row 8(r/4) + 4(l/32) + r%4 of the wave's 32,
// token l%32 of column tile ct).  NaN cells first take the reference's bits, as
// the plain epilogue's do; then the up tiles go through LDS (the staging slots,
// free after the loop's last barrier) to the gate waves, which form y and its
// Q8_0 block per token: 16 rows in lane l, 16 in lane l ^ 32.
template <int RT, int CT>
__device__ __forceinline__ void swiglu_epilogue(float (&acc)[CT][16], GemmLdsH<RT>& s, const GemmW& gw,
                                                const uint8_t* __restrict__ W, const uint8_t* __restrict__ W2,
                                                const uint8_t* __restrict__ X, int m0, int n0, int m_tokens, int nb,
                                                int nan_mode, int wr, int wc, int lane) {
    constexpr int WCN = 4 / CT, HR = RT / 2;  // waves per row tile, row tiles of each matrix
    static_assert(sizeof(GemmLdsH<RT>) >= (size_t)HR * WCN * CT * 16 * 64 * 4, "up tiles fit the staging LDS");
    const int col = lane & 31, half = lane >> 5;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const bool up = wr >= HR;
    const int tr = up ? wr - HR : wr;  // the row tile within its matrix
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int tok = n0 + wc * 32 * CT + ct * 32 + col;
        bool any_nan = false;
#pragma unroll
        for (int r = 0; r < 16; r++) any_nan |= __builtin_isnan(acc[ct][r]);
        if (any_nan && tok < m_tokens) {
            for (int r = 0; r < 16; r++) {
                const int row = m0 + tr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (__builtin_isnan(acc[ct][r]))
                    acc[ct][r] = s_order_nan_bits((up ? W2 : W) + row * bpr, X + tok * bpr, nb, nan_mode);
            }
        }
    }
    float* U = reinterpret_cast<float*>(&s);  // [tr][wc][ct][r][lane]
    if (up) {
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int r = 0; r < 16; r++) U[(((tr * WCN + wc) * CT + ct) * 16 + r) * 64 + lane] = acc[ct][r];
    }
    __syncthreads();
    if (up) return;
    const int fq = gw.m[0] / 32;  // Q8_0 blocks per token row of y
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int tok = n0 + wc * 32 * CT + ct * 32 + col;
        float y[16];
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float g = acc[ct][r], u = U[(((tr * WCN + wc) * CT + ct) * 16 + r) * 64 + lane];
            y[r] = (g / (1.0f + expf_libm(-g))) * u;
            amax = fmaxf(amax, abs_no_nan(y[r]));
        }
        amax = fmaxf(amax, xor_f(amax, 32));  // the token's other 16 rows
        if (tok >= m_tokens) continue;
        const float d = amax / 127.0f;
        const float id = q8_id(amax);
        uint8_t* yb = gw.yq + ((int64_t)tok * fq + (m0 + tr * 32) / 32) * kQ80Bytes;
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = (uint32_t)(uint8_t)(int8_t)(int)__builtin_rintf(y[4 * g4 + i] * id);
            // rows 8g4 + 4half .. +3: quants at bytes 2 + 8g4 + 4half, 2-byte aligned
            uint16_t* p = reinterpret_cast<uint16_t*>(yb + 2 + 8 * g4 + 4 * half);
            p[0] = (uint16_t)(q[0] | (q[1] << 8));
            p[1] = (uint16_t)(q[2] | (q[3] << 8));
        }
        if (half == 0) *reinterpret_cast<uint16_t*>(yb) = __builtin_bit_cast(uint16_t, (_Float16)d);
    }
}

// SWG: SwiGLU pairs.  w[0] = gate, w[1] = up (m[0] rows each): a workgroup's
// 32RT staged rows are 16RT gate rows and the same up rows, the waves of the up
// rows hand their tiles to the gate rows' waves through LDS, and those write
// Q8_0(y), y = (g / (1 + expf(-g))) * u (bpd_swiglu_fuse_cpu, bench/bpd_cpu.c:5504),
// as k_swiglu does, for each token's 32 consecutive rows; no fp32 output.
template <int RT, int CT, bool SWG = false>
__global__ __launch_bounds__(64 * RT * (4 / CT)) void k_q8_0_gemm_SH(GemmW gw, const uint8_t* __restrict__ X,
                                                                     int m_tokens, int nb, int nan_mode) {
    constexpr int WCN = 4 / CT, NT = 64 * RT * WCN;  // waves per 32-row tile, threads
    static_assert(CT == 1 || CT == 2, "one or two column tiles per wave");
    __shared__ GemmLdsH<RT> s;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wr = wave / WCN, wc = wave % WCN;
    int bx, by;
    sh_tile(blockIdx.x, gw.first[kGemmMulti], (m_tokens + kGT - 1) / kGT, bx, by);
    const int mi = SWG ? 0 : (bx >= gw.first[1]) + (bx >= gw.first[2]);
    const uint8_t* __restrict__ W = gw.w[mi];
    const uint8_t* __restrict__ W2 = SWG ? gw.w[1] : nullptr;
    float* __restrict__ out = gw.out[mi];
    const int m_weight = gw.m[mi];
    const int m0 = (bx - gw.first[mi]) * (SWG ? 16 : 32) * RT, n0 = by * kGT;
    const int64_t bpr = (int64_t)nb * kQ80Bytes;
    const int col = lane & 31, half = lane >> 5;
    const int ra = wr * 32 + col;
    // lanes 32-63 give K indices 8-15 of the scale MFMA: they read the zero rows
    const int za = half ? 32 * RT : ra;
    for (int i = threadIdx.x; i < 2 * kGH; i += NT) {
        s.da[i / kGH][i % kGH][32 * RT] = 0u;
        s.db[i / kGH][i % kGH][kGT] = 0u;
    }

    float acc[CT][16];
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[ct][r] = 0.0f;

    HRaw<RT, NT> raw;
    const int nh = nb / kGH;
    // the f16 scale operands: only dword 0 changes per block, the zeros stay in place
    u32x4h a16 = {0u, 0u, 0u, 0u}, b16[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) b16[ct] = u32x4h{0u, 0u, 0u, 0u};
    half_load<RT, NT>(raw, W, W2, X, m0, n0, m_weight, m_tokens, 0, bpr);
    half_store<RT, NT>(s, 0, raw);
    __syncthreads();

    for (int h = 0; h < nh; h++) {
        const int slot = h & 1;
        if (h + 1 < nh) half_load<RT, NT>(raw, W, W2, X, m0, n0, m_weight, m_tokens, (h + 1) * kGH, bpr);
        // block pairs: the swizzle of the operand reads changes once per pair (the
        // pair loop unrolled, the block loop not: 117.7 against 120.2 us at cfg4;
        // both unrolled spill)
#pragma unroll
        for (int pu = 0; pu < kGH / 2; pu++) {
        const int offa = 16 * (half ^ h_swz(ra, 2 * pu));
        int offb[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) offb[ct] = 16 * (half ^ h_swz(wc * 32 * CT + ct * 32 + col, 2 * pu));
#pragma unroll 1
        for (int u = 2 * pu; u < 2 * pu + 2; u++) {
            const i32x4 fa = *reinterpret_cast<const i32x4*>(&s.qa[slot][u][ra][offa]);
            // scale products RN(Ad*Bd) as a rank-1 f16 MFMA: the f16 scales of lanes 0-31
            // are K index 0 (row / column scale), every other K index is zero, so D is the
            // exact product Ad*Bd (11 x 11 bits) plus zeros; |Ad*Bd| >= 2^-48 or 0, never
            // fp32-subnormal; Inf and NaN scales give the fp32 product's Inf / NaN.  (The
            // fp32 form of the same product, v_mfma_f32_32x32x2f32, takes twice the
            // passes: 134 -> 123 us at cfg4.)
            a16[0] = s.da[slot][u][za];
#pragma unroll
            for (int ct = 0; ct < CT; ct++) {
                const int cb = wc * 32 * CT + ct * 32 + col;
                const i32x4 fb = *reinterpret_cast<const i32x4*>(&s.qb[slot][u][cb][offb[ct]]);
                b16[ct][0] = s.db[slot][u][half ? kGT : cb];
                const i32x16 zero = {0};
                const f32x16 fzero = {0.0f};
                const i32x16 sb = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, zero, 0, 0, 0);
                const f32x16 delta = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(h16x8, a16), __builtin_bit_cast(h16x8, b16[ct]), fzero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float prod = (float)sb[r] * delta[r];
                    acc[ct][r] = acc[ct][r] + prod;
                }
            }
        }
        }
        // the other slot was last read before the previous barrier
        if (h + 1 < nh) half_store<RT, NT>(s, slot ^ 1, raw);
        __syncthreads();
    }

    if constexpr (SWG) {
        swiglu_epilogue<RT, CT>(acc, s, gw, W, W2, X, m0, n0, m_tokens, nb, nan_mode, wr, wc, lane);
        return;
    }
    // register r of lane l is row 8(r/4) + 4(l/32) + r%4 of the tile: runs of 4 rows
    const bool full_rows = m0 + wr * 32 + 32 <= m_weight && (m_weight & 3) == 0;
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int tok = n0 + wc * 32 * CT + ct * 32 + col;
        if (tok >= m_tokens) continue;
        // NaN cells take the reference's bits (rare: only Inf / NaN scales make them)
        bool any_nan = false;
#pragma unroll
        for (int r = 0; r < 16; r++) any_nan |= __builtin_isnan(acc[ct][r]);
        if (any_nan) {
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (row < m_weight && __builtin_isnan(acc[ct][r]))
                    acc[ct][r] = s_order_nan_bits(W + row * bpr, X + tok * bpr, nb, nan_mode);
            }
        }
        float* o = out + (int64_t)tok * m_weight + m0 + wr * 32 + 4 * half;
        if (full_rows) {
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<float4*>(o + 8 * g) =
                    make_float4(acc[ct][4 * g], acc[ct][4 * g + 1], acc[ct][4 * g + 2], acc[ct][4 * g + 3]);
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wr * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (row < m_weight) o[8 * (r >> 2) + (r & 3)] = acc[ct][r];
            }
        }
    }
}

// y = silu(gate) * up in Q8_0 (yq: m_tokens rows of F/32 blocks, not Xq): false
// when the shape does not fit the pair form (F % 64, K % 128, 4-byte alignment).
bool launch_q8_0_gemm_S_swiglu(const uint8_t* Wg, const uint8_t* Wu, int F, const uint8_t* Xq, int m_tokens, int K,
                               int nan_mode, uint8_t* yq, hipStream_t s) {
    constexpr int RT = 4, CT = 2;
    const auto al4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; };
    if (F <= 0 || F % (16 * RT) != 0 || K <= 0 || K % 128 != 0 || m_tokens <= 0 || !al4(Wg) || !al4(Wu) ||
        !al4(Xq))
        return false;
    GemmW g{};
    const int panels = F / (16 * RT);
    for (int i = 0; i < kGemmMulti; i++) {
        g.w[i] = i == 1 ? Wu : Wg;
        g.out[i] = nullptr;
        g.m[i] = F;
        g.first[i] = i == 0 ? 0 : panels;
    }
    g.first[kGemmMulti] = panels;
    g.yq = yq;
    hipLaunchKernelGGL((k_q8_0_gemm_SH<RT, CT, true>), dim3(panels * ((m_tokens + kGT - 1) / kGT)),
                       dim3(64 * RT * (4 / CT)), 0, s, g, Xq, m_tokens, K / 32, nan_mode);
    return true;
}

template <int RT, int CT>
static void launch_sh(const uint8_t* const* W, float* const* out, const int* M, int n, const uint8_t* Xq, int m_tokens,
                      int K, int nan_mode, hipStream_t s) {
    GemmW g{};
    int blocks = 0;
    for (int i = 0; i < kGemmMulti; i++) {
        g.first[i] = blocks;
        if (i < n) {
            g.w[i] = W[i];
            g.out[i] = out[i];
            g.m[i] = M[i];
            blocks += (M[i] + 32 * RT - 1) / (32 * RT);
        } else {
            g.w[i] = W[0];
            g.out[i] = out[0];
            g.m[i] = M[0];
        }
    }
    g.first[kGemmMulti] = blocks;
    hipLaunchKernelGGL((k_q8_0_gemm_SH<RT, CT>), dim3(blocks * ((m_tokens + kGT - 1) / kGT)),
                       dim3(64 * RT * (4 / CT)), 0, s, g, Xq, m_tokens, K / 32, nan_mode);
}

// n <= kGemmMulti matrices (M[i] rows each, M[i] >= 1) sharing the activation rows
// Xq: out[i][token * M[i] + row].
void launch_q8_0_gemm_S_multi(const uint8_t* const* W, float* const* out, const int* M, int n, const uint8_t* Xq,
                              int m_tokens, int K, int nan_mode, hipStream_t s) {
    bool aligned = K % 128 == 0 && (reinterpret_cast<uintptr_t>(Xq) & 3) == 0;
    for (int i = 0; i < n; i++) aligned = aligned && (reinterpret_cast<uintptr_t>(W[i]) & 3) == 0;
    if (K / 32 == 0 || !aligned) {
        for (int i = 0; i < n; i++) {
            if (K / 32 == 0) {  // the kernel indexes block nb-1
                launch_fill_zero(out[i], (int64_t)M[i] * m_tokens, s);
                continue;
            }
            const dim3 grid((M[i] + kGT - 1) / kGT, (m_tokens + kGT - 1) / kGT);
            hipLaunchKernelGGL(k_q8_0_gemm_S, grid, dim3(256), 0, s, W[i], Xq, out[i], M[i], m_tokens, K / 32,
                               nan_mode);
        }
        return;
    }
    // 128 weight rows per workgroup, two 512-thread workgroups per CU.  (224 rows,
    // one 896-thread workgroup per CU, balances cfg4's 14336 rows over 256 CUs
    // exactly but measured slower: 150.9 us vs 146.)  64 or 32 rows when 128
    // leave CUs idle: the 4096-row and 1024-row projections of a 512-token
    // prefill.
    const int tok_tiles = (m_tokens + kGT - 1) / kGT;
    const auto wgs = [&](int rows) {
        int64_t b = 0;
        for (int i = 0; i < n; i++) b += (M[i] + rows - 1) / rows;
        return b * tok_tiles;
    };
    // Waves of 32 rows x 64 tokens at 128 rows, of 32 x 32 below it: a launch with
    // fewer than 256 128-row workgroups has fewer than 2 such waves per SIMD.
    // (A 512-token prefill's 4096-row O and down: 53 and 178 us in 32 x 32 waves,
    // 63 and 221 us in 32 x 64 waves, with bit-identical outputs.)
    if (wgs(128) >= 256)
        launch_sh<4, 2>(W, out, M, n, Xq, m_tokens, K, nan_mode, s);
    else if (wgs(64) >= 256)
        launch_sh<2, 1>(W, out, M, n, Xq, m_tokens, K, nan_mode, s);
    else
        launch_sh<1, 1>(W, out, M, n, Xq, m_tokens, K, nan_mode, s);
}

void launch_q8_0_gemm_S(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K,
                        int nan_mode, hipStream_t s) {
    const uint8_t* w[1] = {Wq};
    float* o[1] = {out};
    const int m[1] = {m_weight};
    launch_q8_0_gemm_S_multi(w, o, m, 1, Xq, m_tokens, K, nan_mode, s);
}

}  // namespace bpdq
