// q4k.hip — Q4_K super-block kernels for gfx950.
//
//   k_dequant_q4k<ORDER>   Q4_K -> fp32, bpd element map or GGUF element map
//   k_qmatmul_q4k_chain    reference-order GEMV with fp32 x (one fp32 chain per row)
//   k_quant_q8k            fp32 -> Q8_K activation blocks
//   k_q4k_q8k_gemv<ORDER,R> Q4_K x Q8_K GEMV, integer sub-block sums + fixed fp32 tree
#include <mutex>

#include "../../include/bpdq.h"
#include "bpdq_device.h"
#include "bpdq_launch.h"
#include "bpdq_math.h"

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
    // Inf or NaN d / dmin (one wave = one block, so the test is uniform): give NaN
    // results the reference's bits (x86 rules for the bpd map, the CUDA kernel's
    // canonical NaN for the GGUF map).
    const uint32_t h = __builtin_amdgcn_readfirstlane(hdr.x);
    if (f16_exp31(h) || f16_exp31(h >> 16)) {
        if (ORDER == 0) {
            v.x = q4k_bpd_nan(v.x, h & 0xFFFFu, h >> 16, sc, nib & 0xFFu);
            v.y = q4k_bpd_nan(v.y, h & 0xFFFFu, h >> 16, sc, (nib >> 8) & 0xFFu);
            v.z = q4k_bpd_nan(v.z, h & 0xFFFFu, h >> 16, sc, (nib >> 16) & 0xFFu);
            v.w = q4k_bpd_nan(v.w, h & 0xFFFFu, h >> 16, sc, nib >> 24);
        } else {
            v.x = __builtin_isnan(v.x) ? __uint_as_float(kCudaNaN) : v.x;
            v.y = __builtin_isnan(v.y) ? __uint_as_float(kCudaNaN) : v.y;
            v.z = __builtin_isnan(v.z) ? __uint_as_float(kCudaNaN) : v.z;
            v.w = __builtin_isnan(v.w) ? __uint_as_float(kCudaNaN) : v.w;
        }
    }
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
// Reference-order GEMV with fp32 x (bench/bpd_quant.c:88-109):
//   y[r] = (((0 + w_0 x_0) + w_1 x_1) + ...) over k in bpd element order,
// each product and each sum rounded once.  The chain is serial by definition,
// so a row costs K dependent adds (~2.5 ns each on this GPU) however it is
// mapped; everything else is kept off that chain.
//
// A workgroup owns 64 rows and has 5 waves.  Waves 1-4 (producers) turn the
// rows' weights into products RN(w_k * x_k), half a Q4_K block (128 elements,
// sub-blocks 4h..4h+3) per chunk: lane (s, r) = (wave-1, lane) takes sub-block
// 4h+s of row r, i.e. one 16-byte qs load for 32 consecutive elements, the
// block header, and x of those 32 elements (wave-uniform: scalar loads).  The
// weight loads run kChainAhead chunks ahead in registers.  The products go to a
// two-slot LDS ring stored [k/4][row][4], so wave 0 (consumer) lane r reads
// its row's next 4 products as one float4 and only adds, in order.  One
// barrier per chunk.  Rows are independent and every product and sum is the
// reference's, so the output is bpd_qmatmul_q4k's bit for bit.
// ----------------------------------------------------------------------------
// The x86 bits of a row whose sum came out NaN.  On x86 the first NaN of the
// chain sticks: sum + p keeps sum's NaN, w*x keeps w's (the reference build
// puts the weight first), and an invalid operation gives the default NaN.  So
// the row's bits are those of its first NaN event, found by running the chain
// again with those rules.  Called only for NaN rows.
__device__ __noinline__ float chain_nan_bits(const uint8_t* __restrict__ rp, const float* __restrict__ x, int nb) {
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
            for (int k = 0; k < 32; k++) {
                const uint32_t q = (qd[(k & 15) >> 2] >> (8 * (k & 3) + (k >= 16 ? 4 : 0))) & 15u;
                const float w = q4k_bpd_nan(fmaf(scale, (float)q, -mn), hdr.x & 0xFFFFu, hdr.x >> 16, sc, q);
                const float xv = xb[32 * j + k];
                float p = w * xv;
                if (__builtin_isnan(p)) p = x86_nan_of(w, xv);
                const float t = sum + p;
                if (__builtin_isnan(t)) return x86_nan_of(sum, p);
                sum = t;
            }
        }
    }
    return sum;
}

constexpr int kChainRows = 64;          // rows per workgroup = consumer lanes
constexpr int kChainWaves = 8;          // 0: consumer (SIMD 0); 4: helps stage x, then exits; others: producers
constexpr int kChainSb = 6;             // sub-blocks (of 32 elements) per chunk: one per producer wave
constexpr int kChainElems = 32 * kChainSb;                        // 192 elements per chunk
constexpr int kChainAhead = 4;          // chunks of weight loads in flight per producer lane
constexpr int kChainRing = 2 * (kChainElems / 4) * kChainRows;  // float4s of the product ring (96 KB)
constexpr int kChainXMax = 16384;       // x staged in LDS up to this K (ring + x <= 160 KB)

// Producer lane's registers for one chunk: its sub-block's block header and 16-byte qs slice.
struct ChainLoad {
    uint4 hdr, qs;
};

__device__ __forceinline__ ChainLoad chain_load(const uint8_t* __restrict__ rp, int c, int p, int nsb) {
    const int sb = min(kChainSb * c + p, nsb - 1);  // sub-blocks past the end repeat the last one (not used)
    const uint8_t* blk = rp + (int64_t)(sb >> 3) * kQ4KBytes;
    return ChainLoad{ld_u128(blk), ld_u128(blk + 16 + 16 * (sb & 7))};
}

// v_cvt_f32_ubyteN: byte N of v as an fp32 (the compiler otherwise extracts it with a
// separate v_bfe_u32 once the byte is known to hold a nibble).
template <int N>
__device__ __forceinline__ float cvt_ubyte(uint32_t v) {
    float r;
    if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    if constexpr (N == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Products RN(RN(scale*q - mn) * x) of 32 elements (one sub-block) into the ring:
// elements 4g..4g+3 take the low (g < 4) or high nibbles of qs dword g & 3.
__device__ __forceinline__ void chain_products(float4* __restrict__ dst, const uint4 qv, const float4 (&xv)[8],
                                               float scale, float mn) {
    const uint32_t qd[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t nib = (g < 4 ? qd[g & 3] : qd[g & 3] >> 4) & 0x0F0F0F0Fu;
        float4 o;
        o.x = fmaf(scale, cvt_ubyte<0>(nib), -mn) * xv[g].x;
        o.y = fmaf(scale, cvt_ubyte<1>(nib), -mn) * xv[g].y;
        o.z = fmaf(scale, cvt_ubyte<2>(nib), -mn) * xv[g].z;
        o.w = fmaf(scale, cvt_ubyte<3>(nib), -mn) * xv[g].w;
        dst[g * kChainRows] = o;
    }
}

// XL: x staged once per workgroup in LDS (K <= kChainXMax), else read from global memory.
template <bool XL>
__global__ __launch_bounds__(64 * kChainWaves) void k_qmatmul_q4k_chain(const uint8_t* __restrict__ w,
                                                                        const float* __restrict__ x,
                                                                        float* __restrict__ y, int M, int nb) {
    constexpr int NT = 64 * kChainWaves;
    constexpr int E4 = kChainElems / 4;
    extern __shared__ __align__(16) float4 chain_lds[];
    float4(*prod)[E4][kChainRows] = reinterpret_cast<float4(*)[E4][kChainRows]>(chain_lds);
    float* xl = reinterpret_cast<float*>(chain_lds + kChainRing);
    const int lane = threadIdx.x & 63;
    // waves go to SIMDs round-robin: 0 and 4 share SIMD 0, the producers take SIMDs 1-3 two each
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = blockIdx.x * kChainRows;
    const int nsb = 8 * nb, nch = (nsb + kChainSb - 1) / kChainSb;
    const int64_t rowbytes = (int64_t)nb * kQ4KBytes;
    const int p = wave < 4 ? wave - 1 : wave - 2;  // producers 1,2,3,5,6,7: sub-block 6c + p of chunk c
    const bool producer = (wave & 3) != 0;
    const uint8_t* rp = w + (int64_t)min(row0 + lane, M - 1) * rowbytes;  // rows past M repeat row M-1
    ChainLoad ring[kChainAhead];
    if (producer) {
#pragma unroll
        for (int a = 0; a < kChainAhead; a++) ring[a] = chain_load(rp, a, p, nsb);
    }
    if (XL) {  // every thread copies x to LDS, 4 loads in flight, while the weight loads are too
        const float4* x4 = reinterpret_cast<const float4*>(x);
        float4* xl4 = reinterpret_cast<float4*>(xl);
        const int n4 = nb * 64;
        for (int i0 = threadIdx.x; i0 < n4; i0 += 4 * NT) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = x4[min(i0 + NT * u, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (i0 + NT * u < n4) xl4[i0 + NT * u] = v[u];
        }
        lds_barrier();
    }
    if (wave == 4) return;  // a finished wave no longer takes part in s_barrier
    if (wave == 0) {
        // the chain: sum = RN(sum + p_k) in element order; chunk c holds elements
        // [192c, 192c + 192) (the last chunk may hold fewer: its tail is never read).
        // Reads go out 12 float4s ahead of the adds.
        float sum = 0.0f;
        for (int c = 0; c < nch; c++) {
            lds_barrier();  // chunk c is in slot c & 1
            const int n4 = min(kChainElems, 32 * (nsb - kChainSb * c)) / 4;
            if (n4 == E4) {
                float4 v[E4];
#pragma unroll
                for (int k4 = 0; k4 < 12; k4++) v[k4] = prod[c & 1][k4][lane];
#pragma unroll
                for (int g = 0; g < E4 / 12; g++) {
                    if (g + 1 < E4 / 12) {
#pragma unroll
                        for (int k4 = 12 * (g + 1); k4 < 12 * (g + 2); k4++) v[k4] = prod[c & 1][k4][lane];
                    }
#pragma unroll
                    for (int k4 = 12 * g; k4 < 12 * (g + 1); k4++) {
                        sum = sum + v[k4].x;
                        sum = sum + v[k4].y;
                        sum = sum + v[k4].z;
                        sum = sum + v[k4].w;
                    }
                }
            } else {
                for (int k4 = 0; k4 < n4; k4++) {
                    const float4 v = prod[c & 1][k4][lane];
                    sum = sum + v.x;
                    sum = sum + v.y;
                    sum = sum + v.z;
                    sum = sum + v.w;
                }
            }
        }
        const int row = row0 + lane;
        if (row < M) y[row] = __builtin_isnan(sum) ? chain_nan_bits(w + (int64_t)row * rowbytes, x, nb) : sum;
        return;
    }
    for (int c0 = 0; c0 < nch; c0 += kChainAhead) {
#pragma unroll
        for (int a = 0; a < kChainAhead; a++) {
            const int c = c0 + a;
            const int sb = kChainSb * c + p;  // wave-uniform
            if (c < nch && sb < nsb) {
                const ChainLoad ld = ring[a];
                // the 8 x reads before the first product write: x and the ring share LDS,
                // so a read after a write could not be moved above it
                const float* xs = (XL ? xl : x) + (int64_t)32 * sb;
                float4 xv[8];
#pragma unroll
                for (int g = 0; g < 8; g++) xv[g] = *reinterpret_cast<const float4*>(xs + 4 * g);
                int sc, m;
                q4k_scale_min(ld.hdr.y, ld.hdr.z, ld.hdr.w, sb & 7, sc, m);
                chain_products(&prod[c & 1][8 * p][lane], ld.qs, xv, f16_ieee(ld.hdr.x) * (float)sc,
                               f16_ieee(ld.hdr.x >> 16) * (float)m);
            }
            // refill the slot after its last use (so the loads can take its registers), on
            // every path, so the count of loads in flight is the same whichever chunks exist
            ring[a] = chain_load(rp, c + kChainAhead, p, nsb);
            // chunk c written: the consumer's barrier c.  Producers and consumer pass
            // exactly nch barriers each; the weight loads of the next chunks stay in flight.
            if (c < nch) lds_barrier();
        }
    }
}

void launch_qmatmul_q4k_chain(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t s) {
    const int nb = K / 256;
    if (nb == 0) {  // the empty sum
        launch_fill_zero(y, M, s);
        return;
    }
    const dim3 grid((M + kChainRows - 1) / kChainRows), block(64 * kChainWaves);
    // more than 64 KB of dynamic LDS is asked for once per process
    static std::once_flag once;
    static bool lds_ok = false;
    std::call_once(once, [] {
        lds_ok = true;
        for (const void* k : {reinterpret_cast<const void*>(&k_qmatmul_q4k_chain<true>),
                              reinterpret_cast<const void*>(&k_qmatmul_q4k_chain<false>)})
            if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
                lds_ok = false;
        (void)hipGetLastError();
    });
    if (!lds_ok) {
        abi_error(BPDQ_ERR_HIP, "bpd_qmatmul_q4k_gpu", "the 96 KB LDS ring of the chain kernel was refused");
        return;
    }
    const bool xl = K <= kChainXMax && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (xl)
        hipLaunchKernelGGL(k_qmatmul_q4k_chain<true>, grid, block, kChainRing * 16 + (size_t)K * 4, s, w, x, y, M,
                           nb);
    else
        hipLaunchKernelGGL(k_qmatmul_q4k_chain<false>, grid, block, kChainRing * 16, s, w, x, y, M, nb);
}

// ----------------------------------------------------------------------------
// bpd_qmm_q4k (bench/bpd_quant.c:114-137): C[r][c] starts at +0.0 and, for k in
// element order, C = RN(RN(B[k][c] * deq(A)[r][k]) + C).  A workgroup takes 4
// rows of A and 256 columns of B: for each Q4_K block its 4 waves dequantize
// one row each into LDS (bpd map, the bits of k_dequant_q4k<0>), then thread c
// runs the 4 chains of its column over the block's 256 k, reading B[k][c]
// coalesced across the wave.  Cells are independent, so each is the
// reference's chain bit for bit; a NaN cell is walked again for the x86 bits of
// its NaN (on x86 the reference keeps the last NaN product: C + p puts p first,
// and B[k][c] * a puts B first).
// ----------------------------------------------------------------------------
__device__ __noinline__ float qmm_nan_bits(const uint8_t* __restrict__ arow, const float* __restrict__ B, int N,
                                           int col, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = arow + (int64_t)b * kQ4KBytes;
        const uint4 hdr = ld_u128(blk);
        const float d = f16_ieee(hdr.x), dmin = f16_ieee(hdr.x >> 16);
        for (int j = 0; j < 8; j++) {
            int sc, m;
            q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
            const float scale = d * (float)sc, mn = dmin * (float)m;
            for (int k = 0; k < 32; k++) {
                const uint32_t q = (blk[16 + 16 * j + (k & 15)] >> (k >= 16 ? 4 : 0)) & 15u;
                const float a = q4k_bpd_nan(fmaf(scale, (float)q, -mn), hdr.x & 0xFFFFu, hdr.x >> 16, sc, q);
                const float bv = B[((int64_t)b * 256 + 32 * j + k) * N + col];
                float p = bv * a;
                if (__builtin_isnan(p)) p = x86_nan_of(bv, a);
                float t = p + acc;
                if (__builtin_isnan(t)) t = x86_nan_of(p, acc);
                acc = t;
            }
        }
    }
    return acc;
}

__global__ __launch_bounds__(256) void k_qmm_q4k(const uint8_t* __restrict__ A, const float* __restrict__ B,
                                                 float* __restrict__ C, int M, int N, int nb) {
    __shared__ __align__(16) float deq[4][256];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r0 = blockIdx.y * 4;
    const int col = blockIdx.x * 256 + t;
    const int cc = min(col, N - 1);  // spare columns repeat column N-1 (not stored)
    const int64_t rowbytes = (int64_t)nb * kQ4KBytes;
    // wave w dequantizes row r0+w (rows past M repeat row M-1); lane l: elements 4l..4l+3
    const uint8_t* arow = A + (int64_t)min(r0 + wave, M - 1) * rowbytes;
    const int j = lane >> 3, dw = 4 * j + (lane & 3), hi = (lane >> 2) & 1;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; b++) {
        const uint8_t* blk = arow + (int64_t)b * kQ4KBytes;
        const uint4 hdr = ld_u128(blk);
        const uint32_t qw = ld_u32(blk + 16 + 4 * dw);
        int sc, m;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
        const float s = f16_ieee(hdr.x) * (float)sc, mn = f16_ieee(hdr.x >> 16) * (float)m;
        const uint32_t nib = (hi ? (qw >> 4) : qw) & 0x0F0F0F0Fu;
        float4 v;
        v.x = fmaf(s, (float)(nib & 0xFFu), -mn);
        v.y = fmaf(s, (float)((nib >> 8) & 0xFFu), -mn);
        v.z = fmaf(s, (float)((nib >> 16) & 0xFFu), -mn);
        v.w = fmaf(s, (float)(nib >> 24), -mn);
        __syncthreads();  // every chain is done with the previous block
        *reinterpret_cast<float4*>(&deq[wave][4 * lane]) = v;
        __syncthreads();
        const float* bp = B + (int64_t)b * 256 * N + cc;
#pragma unroll 4
        for (int k = 0; k < 256; k++) {
            const float bv = bp[(int64_t)k * N];
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = bv * deq[r][k] + acc[r];
        }
    }
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        if (r0 + r >= M) break;
        float v = acc[r];
        if (__builtin_isnan(v)) v = qmm_nan_bits(A + (int64_t)(r0 + r) * rowbytes, B, N, col, nb);
        C[(int64_t)(r0 + r) * N + col] = v;
    }
}

void launch_qmm_q4k(const uint8_t* A, const float* B, float* C, int M, int N, int K, hipStream_t s) {
    if (K / 256 == 0) {  // the empty sum: the reference leaves C at its +0.0 start
        launch_fill_zero(C, (int64_t)M * N, s);
        return;
    }
    hipLaunchKernelGGL(k_qmm_q4k, dim3((N + 255) / 256, (M + 3) / 4), dim3(256), 0, s, A, B, C, M, N, K / 256);
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
    q8k_wave_store(v, y + (int64_t)b * kQ8KBytes, lane);
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

// x operands of chunk c of super-block b, from the Q8_K vector in global
// memory (LX = false) or from the workgroup's LDS copy of it (LX = true: kXS
// bytes per block, qs at 0, the 16 int16 bsums at 256, d at 288).
constexpr int kXS = 304;

template <int ORDER, bool LX>
__device__ __forceinline__ XOps get_x(const uint8_t* __restrict__ xsrc, int b, int c) {
    if (!LX) return load_x<ORDER>(xsrc + (int64_t)b * kQ8KBytes, c);
    const uint8_t* xb = xsrc + b * kXS;
    const int off_lo = ORDER == 0 ? 32 * c : 64 * (c >> 1) + 16 * (c & 1);
    const int off_hi = ORDER == 0 ? 32 * c + 16 : off_lo + 32;
    const uint4 lo = *reinterpret_cast<const uint4*>(xb + off_lo);
    const uint4 hi = *reinterpret_cast<const uint4*>(xb + off_hi);
    const uint32_t bs = *reinterpret_cast<const uint32_t*>(xb + 256 + 4 * c);
    XOps o;
    o.lo[0] = lo.x; o.lo[1] = lo.y; o.lo[2] = lo.z; o.lo[3] = lo.w;
    o.hi[0] = hi.x; o.hi[1] = hi.y; o.hi[2] = hi.z; o.hi[3] = hi.w;
    o.bsum = (int)(int16_t)(bs & 0xFFFFu) + (int)(int16_t)(bs >> 16);
    o.dy = *reinterpret_cast<const float*>(xb + 288);
    return o;
}

// Weight operands of one pass of gemv_rows: qs chunk and header dword of
// G block-groups x R rows.
template <int R, int G>
struct WideW {
    uint4 qv[G][R];
    uint32_t hw[G][R];
};

// PAIR (R = 2): the wave's two rows are row row0 of w and row row0 of w1.
template <int R, int G, bool PAIR = false>
__device__ __forceinline__ void wide_load_g(WideW<R, G>& W, int g, const uint8_t* __restrict__ w, int M, int nb,
                                            int row0, int t0, const uint8_t* __restrict__ w1 = nullptr) {
    const int lane = threadIdx.x & 63;
    const int q = lane >> 3, c = lane & 7;
    const int64_t row_bytes = (int64_t)nb * kQ4KBytes;
    const int b = (t0 + g) * 8 + q;
    const int bb = b < nb ? b : nb - 1;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t* base = PAIR && r == 1 ? w1 : w;
        const int row = PAIR ? row0 : min(row0 + r, M - 1);
        const uint8_t* blk = base + (int64_t)row * row_bytes + (int64_t)bb * kQ4KBytes;
        W.qv[g][r] = ld_u128(blk + 16 + 16 * c);
        W.hw[g][r] = ld_u32(blk + 4 * (c & 3));
    }
}

// One wave's R rows: each pass issues the loads of G block-groups x R rows (a
// 16-byte qs load and a header dword per lane each) before computing any of
// them, so every wave keeps its whole share of the stream in flight.  Rows past
// M reuse row M-1 and slots past nb reuse block nb-1 (their results are
// discarded), so every address stays in the tensors.  row0 < M.  With PRE the
// weights of the first pass were loaded by the caller into `pre`.
//
// PAIR (R = 2): the rows are row0 of w (gate) and row0 of w1 (up), and the
// wave stores y[row0] = (g / (1 + expf(-g))) * u, the SwiGLU of the two
// (bench/bpd_cpu.c:5504-5507) on the bit-exact g and u.
__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf_libm(-g))) * u; }

template <int ORDER, int R, int G, bool LX, bool PRE, bool PAIR = false>
__device__ __forceinline__ void gemv_rows(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xsrc,
                                          float* __restrict__ y, int M, int nb, int row0, const WideW<R, G>& pre,
                                          const uint8_t* __restrict__ w1 = nullptr) {
    const int lane = threadIdx.x & 63;
    const int q = lane >> 3, c = lane & 7;
    const int ngroups = (nb + 7) >> 3;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;

    for (int t0 = 0; t0 < ngroups; t0 += G) {
        WideW<R, G> W;
        XOps x[G];
        bool valid[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int b = (t0 + g) * 8 + q;
            valid[g] = b < nb;
            if (PRE && t0 == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    W.qv[g][r] = pre.qv[g][r];
                    W.hw[g][r] = pre.hw[g][r];
                }
            } else {
                wide_load_g<R, G, PAIR>(W, g, w, M, nb, row0, t0, w1);
            }
            x[g] = get_x<ORDER, LX>(xsrc, valid[g] ? b : nb - 1, c);
        }
        // every load of the pass is issued before any of its data is used
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float cb = block_contrib<ORDER>(bcast_header(W.hw[g][r]), W.qv[g][r], x[g], c);
                if (valid[g]) s[r] = s[r] + cb;
            }
        }
    }
    // slot q lives in lanes 8q..8q+7: row_mirror pairs slots q and q^1, then the
    // four pair sums are lanes 0, 16, 32, 48
    float out[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float v = s[r];
        v = v + dpp_f<0x140>(v);
        const float p01 = readlane_f(v, 0), p23 = readlane_f(v, 16);
        const float p45 = readlane_f(v, 32), p67 = readlane_f(v, 48);
        out[r] = (p01 + p23) + (p45 + p67);
        if (!PAIR && lane == 0 && row0 + r < M) y[row0 + r] = out[r];
    }
    if (PAIR && lane == 0) y[row0] = silu_mul(out[0], out[R - 1]);
}

// ----------------------------------------------------------------------------
// The same GEMV with 4 lanes per super-block: lane (bl = lane/4, c4 = lane%4)
// takes qs chunks c4 and c4+4 of super-block 16t+bl, so the header broadcast,
// the scale decode and the fp32 combine are shared by two chunks and a wave
// pass covers 16 super-blocks.  The qs are loaded as in gemv_rows (instruction
// A: all 8 chunks of blocks 16t..16t+7, B: of blocks 16t+8..16t+15, chunk
// 4(lane/32)+c4) and one v_permlane32_swap per dword pairs them up.  Integer
// sums are the same integers and the fp32 order is the same order, so the
// output equals gemv_rows bit for bit.  Fewer VALU per block pays off on
// shorter matrices and on long rows.
// ----------------------------------------------------------------------------
template <int ORDER>
__device__ __forceinline__ float block4_contrib(const uint4& hdr, const uint32_t (&qd0)[4], const uint32_t (&qd1)[4],
                                                const XOps& x0, const XOps& x1, int c4) {
    int S[4] = {0, 0, 0, 0};  // low and high nibbles of chunks c4 and c4+4
#pragma unroll
    for (int k = 0; k < 4; k++) {
        S[0] = sdot4(qd0[k] & 0x0F0F0F0Fu, x0.lo[k], S[0]);
        S[1] = sdot4((qd0[k] >> 4) & 0x0F0F0F0Fu, x0.hi[k], S[1]);
        S[2] = sdot4(qd1[k] & 0x0F0F0F0Fu, x1.lo[k], S[2]);
        S[3] = sdot4((qd1[k] >> 4) & 0x0F0F0F0Fu, x1.hi[k], S[3]);
    }
    // byte c4 of the scale dwords gives (sc, m) of sub-blocks c4 and c4+4
    const uint32_t a = hdr.y >> (8 * c4), b = hdr.z >> (8 * c4), h = hdr.w >> (8 * c4);
    const int m0 = (int)(b & 63u), m1 = (int)(((h >> 4) & 15u) | ((b >> 2) & 0x30u));
    int isum;
    if (ORDER == 0) {
        const int sc0 = (int)(a & 63u), sc1 = (int)((h & 15u) | ((a >> 2) & 0x30u));
        isum = __mul24(sc0, S[0] + S[1]) + __mul24(sc1, S[2] + S[3]);
    } else {
        // GGUF: chunk c covers halves of sub-blocks 2(c/2) (low) and 2(c/2)+1 (high)
        const int i0 = 2 * (c4 >> 1);
        int s0, s1, s2, s3, unused;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, i0, s0, unused);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, i0 + 1, s1, unused);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, i0 + 4, s2, unused);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, i0 + 5, s3, unused);
        isum = __mul24(s0, S[0]) + __mul24(s1, S[1]) + __mul24(s2, S[2]) + __mul24(s3, S[3]);
    }
    int msum = __mul24(m0, x0.bsum) + __mul24(m1, x1.bsum);
    isum += dpp_i<0xB1>(isum);
    isum += dpp_i<0x4E>(isum);
    msum += dpp_i<0xB1>(msum);
    msum += dpp_i<0x4E>(msum);
    const float dd = f16_ieee(hdr.x) * x0.dy;
    const float dm = f16_ieee(hdr.x >> 16) * x0.dy;
    const float av = dd * (float)isum;
    const float mm = dm * (float)msum;
    return av - mm;
}

// Weight operands of one pass of gemv4_rows.
template <int R>
struct FourW {
    uint4 qa[R], qb[R];
    uint32_t hw[R];
};

template <int R>
__device__ __forceinline__ void four_load(FourW<R>& W, const uint8_t* __restrict__ w, int M, int nb, int row0, int t) {
    const int lane = threadIdx.x & 63;
    const int bl = lane >> 2, c4 = lane & 3;
    const int chunk = 4 * (lane >> 5) + c4;
    const uint32_t row_bytes = (uint32_t)nb * kQ4KBytes;
    const uint32_t boff = (uint32_t)min(16 * t + bl, nb - 1) * kQ4KBytes;
    const uint32_t offA = (uint32_t)min(16 * t + (bl & 7), nb - 1) * kQ4KBytes + 16 + 16 * chunk;
    const uint32_t offB = (uint32_t)min(16 * t + 8 + (bl & 7), nb - 1) * kQ4KBytes + 16 + 16 * chunk;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t* rp = w + (size_t)min(row0 + r, M - 1) * row_bytes;
        W.qa[r] = ld_u128(rp + offA);
        W.qb[r] = ld_u128(rp + offB);
        W.hw[r] = ld_u32(rp + boff + 4 * c4);
    }
}

template <int ORDER, int R, bool LX, bool PRE>
__device__ __forceinline__ void gemv4_rows(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xsrc,
                                           float* __restrict__ y, int M, int nb, int row0, const FourW<R>& pre) {
    const int lane = threadIdx.x & 63;
    const int bl = lane >> 2, c4 = lane & 3;
    const int ngroups = (nb + 15) >> 4;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;

    for (int t = 0; t < ngroups; t++) {
        const int b = 16 * t + bl;
        const bool valid = b < nb, valid_hi = b + 8 < nb;
        FourW<R> W;
        if (PRE && t == 0)
            W = pre;
        else
            four_load<R>(W, w, M, nb, row0, t);
        const int bb = min(b, nb - 1);
        const XOps x0 = get_x<ORDER, LX>(xsrc, bb, c4);
        const XOps x1 = get_x<ORDER, LX>(xsrc, bb, c4 + 4);
        // every load of the pass is issued before any of its data is used
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t qd0[4] = {W.qa[r].x, W.qa[r].y, W.qa[r].z, W.qa[r].w};
            uint32_t qd1[4] = {W.qb[r].x, W.qb[r].y, W.qb[r].z, W.qb[r].w};
#pragma unroll
            for (int k = 0; k < 4; k++) swap32(qd0[k], qd1[k]);
            const float c = block4_contrib<ORDER>(bcast_header(W.hw[r]), qd0, qd1, x0, x1, c4);
            uint32_t c_lo = __float_as_uint(c), c_hi = c_lo;
            swap32(c_lo, c_hi);  // lanes 0-31: c_hi = contribution of block b+8
            float v = s[r];
            if (valid) v = v + c;
            if (valid_hi) v = v + __uint_as_float(c_hi);
            s[r] = v;
        }
    }
    // slot q lives in lanes 4q..4q+3 (q < 8): row_half_mirror pairs slots q and
    // q^1, row_mirror the pairs, and lanes 0 and 16 hold the two halves
#pragma unroll
    for (int r = 0; r < R; r++) {
        float v = s[r];
        v = v + dpp_f<0x141>(v);
        v = v + dpp_f<0x140>(v);
        const float lo = readlane_f(v, 0), hi = readlane_f(v, 16);
        if (lane == 0 && row0 + r < M) y[row0 + r] = lo + hi;
    }
}

// KIND 0: gemv_rows (8 lanes per super-block), KIND 1: gemv4_rows.
template <int KIND, int R, int G>
struct PassW;
template <int R, int G>
struct PassW<0, R, G> { using type = WideW<R, G>; };
template <int R, int G>
struct PassW<1, R, G> { using type = FourW<R>; };

template <int KIND, int R, int G>
__device__ __forceinline__ void load_first(typename PassW<KIND, R, G>::type& W, const uint8_t* __restrict__ w, int M,
                                           int nb, int row0) {
    if constexpr (KIND == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) wide_load_g<R, G>(W, g, w, M, nb, row0, 0);
    } else {
        four_load<R>(W, w, M, nb, row0, 0);
    }
}

template <int KIND, int ORDER, int R, int G, bool LX = false, bool PRE = false>
__device__ __forceinline__ void rows(const uint8_t* __restrict__ w, const uint8_t* __restrict__ xsrc,
                                     float* __restrict__ y, int M, int nb, int row0,
                                     const typename PassW<KIND, R, G>::type& pre) {
    if constexpr (KIND == 0)
        gemv_rows<ORDER, R, G, LX, PRE>(w, xsrc, y, M, nb, row0, pre);
    else
        gemv4_rows<ORDER, R, LX, PRE>(w, xsrc, y, M, nb, row0, pre);
}

// R rows per wave, WPB waves per workgroup.
template <int KIND, int ORDER, int R, int G, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_gemv(const uint8_t* __restrict__ w,
                                                           const uint8_t* __restrict__ xq, float* __restrict__ y,
                                                           int M, int nb) {
    // the wave index is uniform across the wave; saying so keeps row offsets scalar
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (xcd_major(blockIdx.x, gridDim.x) * WPB + wave) * R;
    if (row0 >= M) return;
    typename PassW<KIND, R, G>::type unused;
    rows<KIND, ORDER, R, G>(w, xq, y, M, nb, row0, unused);
}

// ----------------------------------------------------------------------------
// Span GEMV: gemv4_rows's arithmetic with the weights read as contiguous spans.
// A wave owns R rows of K = 256*NB.  Its weight bytes are read as aligned
// 16-byte pieces of one span (JOINT: R consecutive rows of one matrix,
// R*NB*9 pieces) or of R spans (one row each, rows of different matrices),
// lane l loading pieces l, l+64, ..., so that every load instruction covers
// whole 128-byte lines; the loads are non-temporal (every byte is read once)
// and all of them are issued before any compute.  The wave writes the pieces
// to its own LDS slot and reads them back in gemv4_rows's mapping: lane
// (bl, c4) takes qs chunks c4 and c4+4 and the 16-byte header of super-block
// 16t+bl, so a pass covers 16 super-blocks of a row and the header, the scale
// decode and the fp32 combine are shared by 4 lanes.  Passes run row by row,
// each as soon as the loads holding it are in.  Operands, integer sums, the
// valid-block rule and the fp32 order are gemv4_rows's (and so gemv_rows's):
// the bits are the same.  Weights must be 16-byte aligned (rows are then too:
// 144*NB is a multiple of 16 for even NB).
// Measured at 14336x4096 (graph of back-to-back launches over weights beyond
// the MALL): 6.73 us against 7.36 for gemv_rows with per-lane chunk loads; the
// same span in gemv_rows's 8-lane mapping 6.98.
// ----------------------------------------------------------------------------
// PB (pass buffer): instead of a slot holding every load, the wave's LDS holds
// one pass (16 super-blocks, 2,304 bytes), refilled from the staged loads
// before each pass; for long rows, whose spans would not fit LDS at full
// occupancy.
template <int NB, int R, bool JOINT, bool PB = false>
struct Span {
    static constexpr int kSegs = JOINT ? 1 : R;
    static constexpr int kSegPieces = (JOINT ? R : 1) * NB * 9;
    static constexpr int kSegLoads = (kSegPieces + 63) / 64;
    static constexpr int kLoads = kSegs * kSegLoads;
    static constexpr int kSlot = PB ? 16 * kQ4KBytes : kLoads * 1024;  // LDS bytes per wave
    static constexpr int kNT = (NB + 15) / 16;   // passes per row
    // first piece of pass t of row r inside its segment, and the pass's pieces
    static constexpr int pass_first(int r, int t) { return ((JOINT ? r * NB : 0) + 16 * t) * 9; }
    static constexpr int pass_pieces(int t) { return (16 * t + 16 < NB ? 16 : NB - 16 * t) * 9; }
    // loads, in issue order, that hold every piece of pass t of row r
    static constexpr int covering(int r, int t) {
        const int end = 16 * t + 16 < NB ? 16 * t + 16 : NB;
        return JOINT ? ((r * NB + end) * 9 + 63) / 64 : r * kSegLoads + (end * 9 + 63) / 64;
    }
    // LDS offset of row r's first super-block
    static constexpr int row_offset(int r) { return JOINT ? r * NB * kQ4KBytes : r * kSegLoads * 1024; }
};

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// The wave's LDS writes are complete before its later LDS reads are issued (and
// the compiler keeps the accesses in that order).
__device__ __forceinline__ void lds_wave_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Every load of the wave's span(s): segment g starts at seg[g] and has np[g] >= 1
// pieces inside the tensor; lanes past them repeat its last piece.
template <class S>
__device__ __forceinline__ void span_issue(u32x4v (&v)[S::kLoads], const uint8_t* const (&seg)[S::kSegs],
                                           const int (&np)[S::kSegs]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < S::kSegs; g++)
#pragma unroll
        for (int u = 0; u < S::kSegLoads; u++) {
            const uint32_t p = (uint32_t)min(lane + 64 * u, np[g] - 1);
            v[g * S::kSegLoads + u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(seg[g] + 16u * p));
        }
}

// x operands of every pass from the Q8_K vector in global memory (issue these
// before the span loads: the first pass then waits for no weight bytes it does
// not use).
template <int ORDER, int NB>
__device__ __forceinline__ void span_load_x(XOps (&xr)[(NB + 15) / 16][2], const uint8_t* __restrict__ xq) {
    const int lane = threadIdx.x & 63, bl = lane >> 2, c4 = lane & 3;
#pragma unroll
    for (int t = 0; t < (NB + 15) / 16; t++) {
        const uint8_t* xb = xq + (int64_t)min(16 * t + bl, NB - 1) * kQ8KBytes;
        xr[t][0] = load_x<ORDER>(xb, c4);
        xr[t][1] = load_x<ORDER>(xb, c4 + 4);
    }
}

// The R row results (wave-uniform) from the staged loads; x from xr (LX false)
// or from the workgroup's LDS copy xl (LX true).
template <int ORDER, int NB, int R, bool JOINT, bool LX, bool PB = false>
__device__ __forceinline__ void span_rows(const u32x4v (&v)[Span<NB, R, JOINT, PB>::kLoads],
                                          uint8_t* __restrict__ slot, const uint8_t* __restrict__ xl,
                                          const XOps (&xr)[(NB + 15) / 16][2], float (&out)[R]) {
    using S = Span<NB, R, JOINT, PB>;
    const int lane = threadIdx.x & 63, bl = lane >> 2, c4 = lane & 3;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;
    int written = 0;  // loads already in the slot (compile-time after unrolling)
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int t = 0; t < S::kNT; t++) {
            const int b = 16 * t + bl, bb = min(b, NB - 1);
            const uint8_t* blk;
            if constexpr (PB) {
                // the pass's pieces, in order, from the loads of its segment that hold
                // any (the previous pass's reads were consumed before these writes)
                const int g = JOINT ? 0 : r, p0 = S::pass_first(r, t), n = S::pass_pieces(t);
#pragma unroll
                for (int u = 0; u < S::kSegLoads; u++) {
                    if (64 * u + 63 < p0 || 64 * u >= p0 + n) continue;
                    const int q = lane + 64 * u - p0;
                    if (q >= 0 && q < n) *reinterpret_cast<u32x4v*>(slot + 16 * q) = v[g * S::kSegLoads + u];
                }
                lds_wave_order();
                blk = slot + (bb - 16 * t) * kQ4KBytes;
            } else {
                const int need = S::covering(r, t);
#pragma unroll
                for (int u = 0; u < S::kLoads; u++)
                    if (u >= written && u < need) *reinterpret_cast<u32x4v*>(slot + 16 * (lane + 64 * u)) = v[u];
                written = need > written ? need : written;
                lds_wave_order();
                blk = slot + S::row_offset(r) + bb * kQ4KBytes;
            }
            const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
            const uint4 qa = *reinterpret_cast<const uint4*>(blk + 16 + 16 * c4);
            const uint4 qb = *reinterpret_cast<const uint4*>(blk + 80 + 16 * c4);
            const uint32_t qd0[4] = {qa.x, qa.y, qa.z, qa.w};
            const uint32_t qd1[4] = {qb.x, qb.y, qb.z, qb.w};
            float c;
            if constexpr (LX)
                c = block4_contrib<ORDER>(hdr, qd0, qd1, get_x<ORDER, true>(xl, bb, c4),
                                          get_x<ORDER, true>(xl, bb, c4 + 4), c4);
            else
                c = block4_contrib<ORDER>(hdr, qd0, qd1, xr[t][0], xr[t][1], c4);
            uint32_t c_lo = __float_as_uint(c), c_hi = c_lo;
            swap32(c_lo, c_hi);  // lanes 0-31: c_hi = contribution of block b+8
            float acc = s[r];
            if (b < NB) acc = acc + c;
            if (b + 8 < NB) acc = acc + __uint_as_float(c_hi);
            // this pass's arithmetic is done before the next pass's LDS writes, which
            // wait for their loads: without this the compiler hoists those writes
            // (and their vmcnt waits) above it, and every pass waits for every load
            asm volatile("" : "+v"(acc) : : "memory");
            s[r] = acc;
        }
    }
    // slot q lives in lanes 4q..4q+3 (q < 8): row_half_mirror pairs slots q and
    // q^1, row_mirror the pairs, and lanes 0 and 16 hold the two halves
#pragma unroll
    for (int r = 0; r < R; r++) {
        float t = s[r];
        t = t + dpp_f<0x141>(t);
        t = t + dpp_f<0x140>(t);
        out[r] = readlane_f(t, 0) + readlane_f(t, 16);
    }
}

// Single matrix, R consecutive rows per wave, x as Q8_K in global memory.
template <int ORDER, int NB, int R, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_gemv_span(const uint8_t* __restrict__ w,
                                                                const uint8_t* __restrict__ xq,
                                                                float* __restrict__ y, int M) {
    using S = Span<NB, R, true>;
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (xcd_major(blockIdx.x, gridDim.x) * WPB + wave) * R;
    if (row0 >= M) return;
    XOps xr[S::kNT][2];
    span_load_x<ORDER, NB>(xr, xq);
    // rows past M repeat the last piece of row M-1 (their results are not stored)
    const uint8_t* seg[1] = {w + (int64_t)row0 * (NB * kQ4KBytes)};
    const int np[1] = {min(R, M - row0) * NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    float out[R];
    span_rows<ORDER, NB, R, true, false>(v, slots[wave], nullptr, xr, out);
#pragma unroll
    for (int r = 0; r < R; r++)
        if ((threadIdx.x & 63) == 0 && row0 + r < M) y[row0 + r] = out[r];
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
    int safe;  // a matrix with M > 0
    int rows;  // total rows
};

template <int KIND, int ORDER, int R, int G, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_gemv_multi(MultiArgs a, const uint8_t* __restrict__ xq, int nb) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int gw = xcd_major(blockIdx.x, gridDim.x) * WPB + wave;
    int i = 0;
#pragma unroll
    for (int k = 1; k < kMulti; k++)
        if (gw >= a.first[k]) i = k;
    if (gw >= a.first[kMulti]) return;
    const int row0 = (gw - a.first[i]) * R;
    if (row0 >= a.M[i]) return;
    typename PassW<KIND, R, G>::type unused;
    rows<KIND, ORDER, R, G>(a.w[i], xq, a.y[i], a.M[i], nb, row0, unused);
}

// Launch shapes, measured on MI355X (one graph of back-to-back launches over
// weights that do not fit the MALL):
//   kWide  8 lanes/block, 2 rows x 2 block-groups per wave, 4 waves: best for
//          many short rows (14336x4096: 7.37 us vs 7.75 for k4Row2)
//   k4Row1 4 lanes/block, 1 row per wave, 8 waves: best up to ~8K rows of
//          K <= 4096 (4096x4096: 3.87 us vs 4.00; 1024x4096: 2.85 vs 3.05)
//   k4Row2 4 lanes/block, 2 rows per wave, 4 waves: best for long rows
//          (4096x14336: 8.13 us vs 8.57)
enum GemvShape { kWide, k4Row1, k4Row2 };

static GemvShape choose_shape(int rows, int nb) {
    if (nb > 16) return k4Row2;
    return rows <= 8192 ? k4Row1 : kWide;
}

static int shape_rows_per_wave(GemvShape sh) { return sh == k4Row1 ? 1 : 2; }

template <int KIND, int ORDER, int R, int G, int WPB>
static void launch_gemv(const uint8_t* w, const uint8_t* xq, float* y, int M, int nb, hipStream_t s) {
    const int waves = (M + R - 1) / R;
    hipLaunchKernelGGL((k_q4k_q8k_gemv<KIND, ORDER, R, G, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0,
                       s, w, xq, y, M, nb);
}

// Span kernels where they apply (K = 4096, 16-byte aligned weights): two rows
// per wave, one up to 2048 rows (measured: 4096x4096 3.54 us against 3.85 for
// k4Row1, 1024x4096 2.40 against 2.86), 4 waves per workgroup.
static bool span16(int nb, const void* w) { return nb == 16 && (reinterpret_cast<uintptr_t>(w) & 15) == 0; }
static int span_rows_per_wave(int rows) { return rows <= 2048 ? 1 : 2; }

template <int ORDER, int R>
static void launch_span(const uint8_t* w, const uint8_t* xq, float* y, int M, hipStream_t s) {
    constexpr int WPB = 4;
    const int waves = (M + R - 1) / R;
    hipLaunchKernelGGL((k_q4k_q8k_gemv_span<ORDER, 16, R, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0, s,
                       w, xq, y, M);
}

template <int ORDER>
static void launch_gemv_order(const uint8_t* w, const uint8_t* xq, float* y, int M, int nb, hipStream_t s) {
    if (span16(nb, w)) {
        if (span_rows_per_wave(M) == 1) launch_span<ORDER, 1>(w, xq, y, M, s); else launch_span<ORDER, 2>(w, xq, y, M, s);
        return;
    }
    switch (choose_shape(M, nb)) {
        case kWide: launch_gemv<0, ORDER, 2, 2, 4>(w, xq, y, M, nb, s); break;
        case k4Row1: launch_gemv<1, ORDER, 1, 1, 8>(w, xq, y, M, nb, s); break;
        case k4Row2: launch_gemv<1, ORDER, 2, 1, 4>(w, xq, y, M, nb, s); break;
    }
}

void launch_qmatmul_q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s) {
    const int nb = K / 256;
    if (order == 0)
        launch_gemv_order<0>(w, xq, y, M, nb, s);
    else
        launch_gemv_order<1>(w, xq, y, M, nb, s);
}

template <int KIND, int ORDER, int R, int G, int WPB>
static void launch_multi(const MultiArgs& a, const uint8_t* xq, int nb, hipStream_t s) {
    const int waves = a.first[kMulti];
    hipLaunchKernelGGL((k_q4k_q8k_gemv_multi<KIND, ORDER, R, G, WPB>), dim3((waves + WPB - 1) / WPB),
                       dim3(64 * WPB), 0, s, a, xq, nb);
}

template <int ORDER>
static void launch_multi_order(const MultiArgs& a, GemvShape sh, const uint8_t* xq, int nb, hipStream_t s) {
    switch (sh) {
        case kWide: launch_multi<0, ORDER, 2, 2, 4>(a, xq, nb, s); break;
        case k4Row1: launch_multi<1, ORDER, 1, 1, 8>(a, xq, nb, s); break;
        case k4Row2: launch_multi<1, ORDER, 2, 1, 4>(a, xq, nb, s); break;
    }
}

static int total_rows(const int* M, int n) {
    int rows = 0;
    for (int i = 0; i < n; i++) rows += M[i];
    return rows;
}

// Wave numbering of a multi launch with R rows per wave.
static MultiArgs make_multi_args(const uint8_t* const* w, float* const* y, const int* M, int n, int R) {
    MultiArgs a;
    a.rows = 0;
    a.safe = 0;
    for (int i = 0; i < n; i++) {
        a.rows += M[i];
        if (M[i] > 0 && M[a.safe] == 0) a.safe = i;
    }
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
    return a;
}

// ----------------------------------------------------------------------------
// GEMV with the Q8_K quantization of an fp32 x fused in: every workgroup
// quantizes all of x into LDS (the same arithmetic as k_quant_q8k, so the
// Q8_K bytes are identical), then runs the GEMV of its rows reading x from LDS.
// Order of work per wave: issue the fp32 x loads of its quantization share,
// issue the weight loads of its first pass, quantize as soon as x arrives
// (x loads were issued first, so waiting for them does not wait for the
// weights), barrier, GEMV.  The weight stream is in flight while x is
// quantized, so the quantization hides behind HBM latency instead of costing
// a launch.  y equals quant_q8_k followed by the Q8_K GEMV bit for bit.
//
// Quantization share: 16 lanes per Q8_K block (the block is one DPP row), lane
// li holds elements 16li..16li+15 = bsum group li; a workgroup covers 4*WPB
// blocks per iteration, IT iterations.
// ----------------------------------------------------------------------------
template <int IT>
struct XPre {
    float4 v[IT][4];
};

template <int WPB, int IT>
__device__ __forceinline__ void x32_load(XPre<IT>& P, const float* __restrict__ x, int nb) {
    const int tid = threadIdx.x, gq = tid >> 4, li = tid & 15;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int b = min(it * 4 * WPB + gq, nb - 1);
        const float* xb = x + (int64_t)b * 256 + 16 * li;
#pragma unroll
        for (int k = 0; k < 4; k++) P.v[it][k] = *reinterpret_cast<const float4*>(xb + 4 * k);
    }
}

template <int WPB, int IT>
__device__ __forceinline__ void x32_quantize(const XPre<IT>& P, uint8_t* __restrict__ xl, int nb) {
    const int tid = threadIdx.x, gq = tid >> 4, li = tid & 15;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int b = it * 4 * WPB + gq;
        float e[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            e[4 * k] = P.v[it][k].x;
            e[4 * k + 1] = P.v[it][k].y;
            e[4 * k + 2] = P.v[it][k].z;
            e[4 * k + 3] = P.v[it][k].w;
        }
        float amax = abs_no_nan(e[0]);
#pragma unroll
        for (int k = 1; k < 16; k++) amax = fmaxf(amax, abs_no_nan(e[k]));
        amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
        amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
        amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror
        amax = fmaxf(amax, dpp_f<0x140>(amax));  // row_mirror: the whole 16-lane row
        const float d = amax / 127.0f;
        const float id = q8_id(amax);
        uint32_t pk[4] = {0u, 0u, 0u, 0u};
        int bsum = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int qv = (int)__builtin_rintf(e[k] * id);
            bsum += qv;
            pk[k >> 2] |= (uint32_t)(qv & 0xFF) << (8 * (k & 3));
        }
        if (b < nb) {
            uint8_t* xb = xl + b * kXS;
            *reinterpret_cast<uint4*>(xb + 16 * li) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            *reinterpret_cast<int16_t*>(xb + 256 + 2 * li) = (int16_t)bsum;
            if (li == 0) *reinterpret_cast<float*>(xb + 288) = d;
        }
    }
}

// Matrix index and first row of wave gw in a MultiArgs launch; waves past the
// last row get (safe, 0) so that their first-pass loads stay in a real tensor.
__device__ __forceinline__ bool wave_rows(const MultiArgs& a, int gw, int R, int& i, int& row0) {
    i = 0;
#pragma unroll
    for (int k = 1; k < kMulti; k++)
        if (gw >= a.first[k]) i = k;
    row0 = (gw - a.first[i]) * R;
    const bool has = gw < a.first[kMulti] && row0 < a.M[i];
    if (!has) {
        i = a.safe;
        row0 = 0;
    }
    return has;
}

template <int KIND, int ORDER, int R, int G, int WPB, int IT>
__global__ __launch_bounds__(64 * WPB) void k_q4k_fused_gemv(MultiArgs a, const float* __restrict__ x, int nb) {
    extern __shared__ __align__(16) uint8_t xl[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int i, row0;
    const bool has = wave_rows(a, xcd_major(blockIdx.x, gridDim.x) * WPB + wave, R, i, row0);
    XPre<IT> P;
    x32_load<WPB, IT>(P, x, nb);
    typename PassW<KIND, R, G>::type pre;
    load_first<KIND, R, G>(pre, a.w[i], a.M[i], nb, row0);
    __builtin_amdgcn_sched_barrier(0);
    x32_quantize<WPB, IT>(P, xl, nb);
    __syncthreads();
    if (!has) return;
    rows<KIND, ORDER, R, G, true, true>(a.w[i], xl, a.y[i], a.M[i], nb, row0, pre);
}

template <int KIND, int ORDER, int R, int G, int WPB, int IT>
static void launch_fused(const MultiArgs& a, const float* x, int nb, hipStream_t s) {
    const int waves = a.first[kMulti];
    hipLaunchKernelGGL((k_q4k_fused_gemv<KIND, ORDER, R, G, WPB, IT>), dim3((waves + WPB - 1) / WPB),
                       dim3(64 * WPB), (size_t)nb * kXS, s, a, x, nb);
}

// Gate and up in one launch with SwiGLU in the epilogue: wave w computes row w
// of both matrices (the 8-lane kernel, two rows per wave) from the shared
// fp32 x, quantized to Q8_K in LDS as in k_q4k_fused_gemv, and stores
// y[w] = silu(gate_w) * up_w.  gate_w and up_w are the bits the plain GEMV
// gives, so y equals the GEMVs followed by bpd_swiglu_fuse_cpu's arithmetic.
// QX: x is already Q8_K (xq), read from global memory, with no quantization pass.
template <int ORDER, int G, int WPB, bool QX = false>
__global__ __launch_bounds__(64 * WPB) void k_q4k_fused_swiglu(const uint8_t* __restrict__ wg,
                                                              const uint8_t* __restrict__ wu, float* __restrict__ y,
                                                              int M, const float* __restrict__ x,
                                                              const uint8_t* __restrict__ xq, int nb) {
    extern __shared__ __align__(16) uint8_t xl[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = xcd_major(blockIdx.x, gridDim.x) * WPB + wave;
    const bool has = row < M;
    const int row0 = has ? row : 0;
    if constexpr (QX) {
        if (!has) return;
        WideW<2, G> pre;
#pragma unroll
        for (int g = 0; g < G; g++) wide_load_g<2, G, true>(pre, g, wg, M, nb, row0, 0, wu);
        gemv_rows<ORDER, 2, G, false, true, true>(wg, xq, y, M, nb, row0, pre, wu);
    } else {
        XPre<1> P;
        x32_load<WPB, 1>(P, x, nb);
        WideW<2, G> pre;
#pragma unroll
        for (int g = 0; g < G; g++) wide_load_g<2, G, true>(pre, g, wg, M, nb, row0, 0, wu);
        __builtin_amdgcn_sched_barrier(0);
        x32_quantize<WPB, 1>(P, xl, nb);
        __syncthreads();
        if (!has) return;
        gemv_rows<ORDER, 2, G, true, true, true>(wg, xl, y, M, nb, row0, pre, wu);
    }
}

template <int ORDER, int WPB>
static void launch_swiglu(const uint8_t* wg, const uint8_t* wu, float* y, int M, const float* x, int nb,
                          hipStream_t s) {
    hipLaunchKernelGGL((k_q4k_fused_swiglu<ORDER, 2, WPB>), dim3((M + WPB - 1) / WPB), dim3(64 * WPB),
                       (size_t)nb * kXS, s, wg, wu, y, M, x, nullptr, nb);
}

// ----------------------------------------------------------------------------
// Span forms (see span_rows) of the multi-matrix, fused-quantization and
// Q8_K gate/up SwiGLU launches, for K = 4096 and 16-byte aligned weights.
// Waves, rows and outputs are numbered as in the kernels above, and so are the
// bits.
// ----------------------------------------------------------------------------
template <int ORDER, int NB, int R, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_q8k_multi_span(MultiArgs a, const uint8_t* __restrict__ xq) {
    using S = Span<NB, R, true>;
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int i, row0;
    if (!wave_rows(a, xcd_major(blockIdx.x, gridDim.x) * WPB + wave, R, i, row0)) return;
    XOps xr[S::kNT][2];
    span_load_x<ORDER, NB>(xr, xq);
    const uint8_t* seg[1] = {a.w[i] + (int64_t)row0 * (NB * kQ4KBytes)};
    const int np[1] = {min(R, a.M[i] - row0) * NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    float out[R];
    span_rows<ORDER, NB, R, true, false>(v, slots[wave], nullptr, xr, out);
#pragma unroll
    for (int r = 0; r < R; r++)
        if ((threadIdx.x & 63) == 0 && row0 + r < a.M[i]) a.y[i][row0 + r] = out[r];
}

// Fused quantization: the workgroup quantizes x into LDS (x32_load /
// x32_quantize, issued before and run after the span loads), then every wave
// runs its rows with x from LDS.
template <int ORDER, int NB, int R, int WPB, bool PB = false>
__global__ __launch_bounds__(64 * WPB) void k_q4k_fused_span(MultiArgs a, const float* __restrict__ x) {
    using S = Span<NB, R, true, PB>;
    constexpr int IT = (NB + 4 * WPB - 1) / (4 * WPB);
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    __shared__ __align__(16) uint8_t xl[NB * kXS];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int i, row0;
    const bool has = wave_rows(a, xcd_major(blockIdx.x, gridDim.x) * WPB + wave, R, i, row0);
    XPre<IT> P;
    x32_load<WPB, IT>(P, x, NB);
    const uint8_t* seg[1] = {a.w[i] + (int64_t)row0 * (NB * kQ4KBytes)};
    const int np[1] = {min(R, a.M[i] - row0) * NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    __builtin_amdgcn_sched_barrier(0);
    x32_quantize<WPB, IT>(P, xl, NB);
    __syncthreads();
    if (!has) return;
    XOps unused[S::kNT][2];
    float out[R];
    span_rows<ORDER, NB, R, true, true, PB>(v, slots[wave], xl, unused, out);
#pragma unroll
    for (int r = 0; r < R; r++)
        if ((threadIdx.x & 63) == 0 && row0 + r < a.M[i]) a.y[i][row0 + r] = out[r];
}

// Gate row r and up row r per wave (two spans) from the Q8_K activation xq,
// y[r] = silu(gate_r) * up_r (k_q4k_fused_swiglu<..., QX = true>'s bits).
template <int ORDER, int NB, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_swiglu_span(const uint8_t* __restrict__ wg,
                                                             const uint8_t* __restrict__ wu, float* __restrict__ y,
                                                             int M, const uint8_t* __restrict__ xq) {
    using S = Span<NB, 2, false>;
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = xcd_major(blockIdx.x, gridDim.x) * WPB + wave;
    if (row >= M) return;
    XOps xr[S::kNT][2];
    span_load_x<ORDER, NB>(xr, xq);
    const int64_t off = (int64_t)row * (NB * kQ4KBytes);
    const uint8_t* seg[2] = {wg + off, wu + off};
    const int np[2] = {NB * 9, NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    float out[2];
    span_rows<ORDER, NB, 2, false, false>(v, slots[wave], nullptr, xr, out);
    if ((threadIdx.x & 63) == 0) y[row] = silu_mul(out[0], out[1]);
}

static bool all_aligned16(const uint8_t* const* w, int n) {
    for (int i = 0; i < n; i++)
        if (reinterpret_cast<uintptr_t>(w[i]) & 15) return false;
    return true;
}

template <int ORDER, int R>
static void launch_multi_span(const MultiArgs& a, const uint8_t* xq, hipStream_t s) {
    constexpr int WPB = 4;
    const int waves = a.first[kMulti];
    hipLaunchKernelGGL((k_q4k_q8k_multi_span<ORDER, 16, R, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0,
                       s, a, xq);
}

void launch_qmatmul_q4k_q8k_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const uint8_t* xq,
                                  int K, int order, hipStream_t s) {
    const int nb = K / 256;
    if (nb == 16 && all_aligned16(w, n)) {
        const int R = span_rows_per_wave(total_rows(M, n));
        const MultiArgs a = make_multi_args(w, y, M, n, R);
        if (a.first[kMulti] == 0) return;
        if (order == 0)
            R == 1 ? launch_multi_span<0, 1>(a, xq, s) : launch_multi_span<0, 2>(a, xq, s);
        else
            R == 1 ? launch_multi_span<1, 1>(a, xq, s) : launch_multi_span<1, 2>(a, xq, s);
        return;
    }
    const GemvShape sh = choose_shape(total_rows(M, n), nb);
    const MultiArgs a = make_multi_args(w, y, M, n, shape_rows_per_wave(sh));
    if (a.first[kMulti] == 0) return;
    if (order == 0)
        launch_multi_order<0>(a, sh, xq, nb, s);
    else
        launch_multi_order<1>(a, sh, xq, nb, s);
}

// Gate and up from a Q8_K activation (K <= 4096), as launch_qmatmul_q4k_fused_swiglu
// computes them after quantizing.
template <int ORDER>
static void launch_swiglu_span(const uint8_t* wg, const uint8_t* wu, float* y, int M, const uint8_t* xq,
                               hipStream_t s) {
    constexpr int WPB = 4;
    hipLaunchKernelGGL((k_q4k_swiglu_span<ORDER, 16, WPB>), dim3((M + WPB - 1) / WPB), dim3(64 * WPB), 0, s, wg, wu, y,
                       M, xq);
}

void launch_qmatmul_q4k_swiglu_q8k(const uint8_t* wg, const uint8_t* wu, float* y, int M, const uint8_t* xq, int K,
                                   int order, hipStream_t s) {
    const int nb = K / 256;
    const uint8_t* wgu[2] = {wg, wu};
    if (nb == 16 && all_aligned16(wgu, 2)) {
        if (order == 0) launch_swiglu_span<0>(wg, wu, y, M, xq, s); else launch_swiglu_span<1>(wg, wu, y, M, xq, s);
        return;
    }
    if (order == 0)
        hipLaunchKernelGGL((k_q4k_fused_swiglu<0, 2, 4, true>), dim3((M + 3) / 4), dim3(256), 0, s, wg, wu, y, M,
                           nullptr, xq, nb);
    else
        hipLaunchKernelGGL((k_q4k_fused_swiglu<1, 2, 4, true>), dim3((M + 3) / 4), dim3(256), 0, s, wg, wu, y, M,
                           nullptr, xq, nb);
}

// One quantization pass covers 4*WPB blocks: 4 waves up to K = 4096, 16 up to
// fused_max_k().
void launch_qmatmul_q4k_fused_swiglu(const uint8_t* wg, const uint8_t* wu, float* y, int M, const float* x, int K,
                                     int order, hipStream_t s) {
    const int nb = K / 256;
    if (nb <= 16) {
        if (order == 0) launch_swiglu<0, 4>(wg, wu, y, M, x, nb, s); else launch_swiglu<1, 4>(wg, wu, y, M, x, nb, s);
    } else {
        if (order == 0) launch_swiglu<0, 16>(wg, wu, y, M, x, nb, s); else launch_swiglu<1, 16>(wg, wu, y, M, x, nb, s);
    }
}

// Fused shapes, measured on MI355X for the decode-chain GEMVs (one graph of
// back-to-back launches, weights beyond the MALL): K <= 4096 takes the 8-lane
// kernel with 4 waves (QKV 6144x4096: 5.14 us vs 5.44 for k4Row1; O 4096x4096:
// 4.36 vs 4.40; gate+up 2x14336x4096: 14.24), longer rows the 4-lane kernel
// with one row per wave and 16 waves (4096x14336: 9.20 us vs 9.50 for 2 rows x
// 8 waves).  IT = 1: 4*WPB Q8_K blocks per quantization pass cover nb.
int fused_max_k() { return 64 * 256; }

// K = 4096: 4 waves per workgroup; from 16,384 rows (gate + up) 8 waves with the
// pass buffer, which halves the workgroups that each quantize x (measured:
// gate+up 2x14336 12.98 us against 13.35; Q/K/V and O 4.9 and 4.1 us against 5.4
// and 4.3 with 8 waves).
template <int ORDER, int R>
static void launch_fused_span(const MultiArgs& a, const float* x, hipStream_t s) {
    const int waves = a.first[kMulti];
    if (R == 2 && a.rows >= 16384) {
        constexpr int WPB = 8;
        hipLaunchKernelGGL((k_q4k_fused_span<ORDER, 16, 2, WPB, true>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB),
                           0, s, a, x);
        return;
    }
    constexpr int WPB = 4;
    hipLaunchKernelGGL((k_q4k_fused_span<ORDER, 16, R, WPB>), dim3((waves + WPB - 1) / WPB), dim3(64 * WPB), 0, s, a,
                       x);
}

void launch_qmatmul_q4k_fused_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const float* x,
                                    int K, int order, hipStream_t s) {
    const int nb = K / 256;
    if (nb == 16 && all_aligned16(w, n)) {
        const int R = span_rows_per_wave(total_rows(M, n));
        const MultiArgs a = make_multi_args(w, y, M, n, R);
        if (a.first[kMulti] == 0) return;
        if (order == 0)
            R == 1 ? launch_fused_span<0, 1>(a, x, s) : launch_fused_span<0, 2>(a, x, s);
        else
            R == 1 ? launch_fused_span<1, 1>(a, x, s) : launch_fused_span<1, 2>(a, x, s);
        return;
    }
    if (nb == 56 && all_aligned16(w, n)) {  // K = 14336: one row per wave through a pass buffer
        constexpr int WPB = 8;
        const MultiArgs a = make_multi_args(w, y, M, n, 1);
        if (a.first[kMulti] == 0) return;
        const dim3 grid((a.first[kMulti] + WPB - 1) / WPB);
        if (order == 0)
            hipLaunchKernelGGL((k_q4k_fused_span<0, 56, 1, WPB, true>), grid, dim3(64 * WPB), 0, s, a, x);
        else
            hipLaunchKernelGGL((k_q4k_fused_span<1, 56, 1, WPB, true>), grid, dim3(64 * WPB), 0, s, a, x);
        return;
    }
    const bool wide = nb <= 16;
    const MultiArgs a = make_multi_args(w, y, M, n, wide ? 2 : 1);
    if (a.first[kMulti] == 0) return;
    if (order == 0) {
        if (wide) launch_fused<0, 0, 2, 2, 4, 1>(a, x, nb, s); else launch_fused<1, 0, 1, 1, 16, 1>(a, x, nb, s);
    } else {
        if (wide) launch_fused<0, 1, 2, 2, 4, 1>(a, x, nb, s); else launch_fused<1, 1, 1, 1, 16, 1>(a, x, nb, s);
    }
}


// ----------------------------------------------------------------------------
// RMSNorm folded into the decode step's GEMVs (n_embd = 4096).  The reference
// runs x = x + y, then h = rmsnorm(x) * w (bpd_add_f32_cpu, bench/bpd_cpu.c:5466;
// bpd_rmsnorm_llama_cpu, :4959-4986) between the O / down projections and the
// Q/K/V / gate-up projections.  Here:
//   - the producer GEMV (O, down) adds each of its rows into the residual row,
//     x[r] = x[r] + y_r, and each workgroup stores the binary64 sum of
//     (double)x[r]^2 over its rows, in row order, as one partial;
//   - the consumer GEMV (Q/K/V, gate/up) sums the partials in a fixed order (so
//     every workgroup gets the same S), and takes mean = (float)(S / n) when
//     (S - E)/n and (S + E)/n, E = 4 n 2^-53 S, round to the same float: any
//     summation order of n non-negative terms is within (n - 1) 2^-53 S of the
//     exact sum, so rounding monotonicity pins the reference's sequential mean
//     to that float; otherwise thread 0 redoes the reference's sequential sum
//     over the row.  Then scale = 1 / sqrtf(mean + eps), h = (x * scale) * w,
//     quantized to Q8_K in LDS exactly as the fused kernels quantize x.
// The arithmetic is k_residual_rmsnorm's, so the Q8_K bytes and every output
// are the same bits as the separate norm launch followed by the GEMV.
// ----------------------------------------------------------------------------

// A thread's first kPartRegs strided partials, loaded before the weight span so
// that waiting for them does not wait for the span (vector loads complete in
// issue order).  The producers write at most 1024 partials (n_embd 4096 rows).
constexpr int kPartRegs = 4;
template <int WPB>
__device__ __forceinline__ void part_load(double (&pp)[kPartRegs], const NormIn& nin) {
#pragma unroll
    for (int k = 0; k < kPartRegs; k++) {
        // every load unconditional (past npart: a re-read of the last partial, then
        // 0), so none is waited for before the next is issued
        const int i = threadIdx.x + k * 64 * WPB;
        const double v = nin.part[min(i, max(nin.npart - 1, 0))];
        pp[k] = i < nin.npart ? v : 0.0;
    }
}

// Binary64 sum of the partials (a thread's strided terms in order, then the
// wave's lanes by xor steps, then the waves in order), the mean and the scale.
// Any order serves: the mean is either pinned by the error bound or recomputed
// sequentially.  Every thread returns the scale.  red: LDS, one double per wave + 1.
template <int WPB>
__device__ __forceinline__ float norm_scale(const double (&pp)[kPartRegs], const NormIn& nin, int n, double* red) {
    const int tid = threadIdx.x;
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < kPartRegs; k++) s += pp[k];
    for (int i = tid + kPartRegs * 64 * WPB; i < nin.npart; i += 64 * WPB) s += nin.part[i];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        double S = 0.0;
        for (int i = 0; i < WPB; i++) S += red[i];
        reinterpret_cast<float*>(red)[2 * WPB] = rms_scale(S, nin.x, n, nin.eps);
    }
    __syncthreads();
    return reinterpret_cast<const float*>(red)[2 * WPB];
}

// The norm weight of x32_load's elements.
template <int WPB, int IT>
__device__ __forceinline__ void w32_load(XPre<IT>& P, const float* __restrict__ w, int nb) {
    x32_load<WPB, IT>(P, w, nb);
}

// h = (x * scale) * w in place of x.
template <int IT>
__device__ __forceinline__ void x32_normalize(XPre<IT>& P, const XPre<IT>& W, float scale) {
#pragma unroll
    for (int it = 0; it < IT; it++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 x = P.v[it][k], w = W.v[it][k];
            P.v[it][k] = make_float4((x.x * scale) * w.x, (x.y * scale) * w.y, (x.z * scale) * w.z,
                                     (x.w * scale) * w.w);
        }
}

// The producer's epilogue: lane 0 of each wave adds its rows into x and squares
// them; the workgroup's partial goes to part[blockIdx.x].  Every wave calls it
// (has = false: no rows).  red: LDS, one double per wave.
template <int R, int WPB>
__device__ __forceinline__ void res_epilogue(const ResOut& ro, const float (&out)[R], int row0, int M, bool has,
                                             double* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double sq = 0.0;
    if (lane == 0 && has) {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (row0 + r < M) {
                const float xn = ro.x[row0 + r] + out[r];
                ro.x[row0 + r] = xn;
                sq += (double)xn * (double)xn;
            }
    }
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
        double p = 0.0;
        for (int i = 0; i < WPB; i++) p += red[i];
        ro.part[blockIdx.x] = p;
    }
}

// Q/K/V (MultiArgs over up to 4 matrices) with the norm in the quantization
// prologue; k_q4k_fused_span otherwise.
template <int ORDER, int R, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_norm_span(MultiArgs a, NormIn nin) {
    constexpr int NB = 16, IT = (NB + 4 * WPB - 1) / (4 * WPB);
    using S = Span<NB, R, true>;
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    __shared__ __align__(16) uint8_t xl[NB * kXS];
    __shared__ double red[WPB + 1];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int i, row0;
    const bool has = wave_rows(a, xcd_major(blockIdx.x, gridDim.x) * WPB + wave, R, i, row0);
    XPre<IT> P, Wn;
    double pp[kPartRegs];
    part_load<WPB>(pp, nin);
    x32_load<WPB, IT>(P, nin.x, NB);
    w32_load<WPB, IT>(Wn, nin.w, NB);
    const uint8_t* seg[1] = {a.w[i] + (int64_t)row0 * (NB * kQ4KBytes)};
    const int np[1] = {min(R, a.M[i] - row0) * NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    __builtin_amdgcn_sched_barrier(0);
    const float scale = norm_scale<WPB>(pp, nin, NB * 256, red);
    x32_normalize<IT>(P, Wn, scale);
    x32_quantize<WPB, IT>(P, xl, NB);
    __syncthreads();
    if (!has) return;
    XOps unused[S::kNT][2];
    float out[R];
    span_rows<ORDER, NB, R, true, true>(v, slots[wave], xl, unused, out);
#pragma unroll
    for (int r = 0; r < R; r++)
        if ((threadIdx.x & 63) == 0 && row0 + r < a.M[i]) a.y[i][row0 + r] = out[r];
}

// O and down: k_q4k_fused_span's rows with the residual epilogue in place of
// the y stores.
template <int ORDER, int NB, int R, int WPB, bool PB>
__global__ __launch_bounds__(64 * WPB) void k_q4k_res_span(const uint8_t* __restrict__ w, int M,
                                                          const float* __restrict__ x, ResOut ro) {
    using S = Span<NB, R, true, PB>;
    constexpr int IT = (NB + 4 * WPB - 1) / (4 * WPB);
    __shared__ __align__(16) uint8_t slots[WPB][S::kSlot];
    __shared__ __align__(16) uint8_t xl[NB * kXS];
    __shared__ double red[WPB];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0w = (xcd_major(blockIdx.x, gridDim.x) * WPB + wave) * R;
    const bool has = row0w < M;
    const int row0 = has ? row0w : 0;
    XPre<IT> P;
    x32_load<WPB, IT>(P, x, NB);
    const uint8_t* seg[1] = {w + (int64_t)row0 * (NB * kQ4KBytes)};
    const int np[1] = {min(R, M - row0) * NB * 9};
    u32x4v v[S::kLoads];
    span_issue<S>(v, seg, np);
    __builtin_amdgcn_sched_barrier(0);
    x32_quantize<WPB, IT>(P, xl, NB);
    __syncthreads();
    float out[R];
    if (has) {
        XOps unused[S::kNT][2];
        span_rows<ORDER, NB, R, true, true, PB>(v, slots[wave], xl, unused, out);
    }
    res_epilogue<R, WPB>(ro, out, row0, M, has, red);
}

// Launch shapes: Q/K/V and O as launch_fused_span picks them (4 waves, R rows per
// wave), gate/up as launch_swiglu_span (4 waves), down (K = 14336) as
// launch_qmatmul_q4k_fused_multi (8 waves, one row per wave through a pass buffer).
bool norm_fusion_fits(int n_embd, int ff) { return n_embd == 4096 && (ff == 4096 || ff == 14336); }

template <int ORDER, int R>
static void launch_norm_span(const MultiArgs& a, const NormIn& nin, hipStream_t s) {
    constexpr int WPB = 4;
    hipLaunchKernelGGL((k_q4k_norm_span<ORDER, R, WPB>), dim3((a.first[kMulti] + WPB - 1) / WPB), dim3(64 * WPB), 0,
                       s, a, nin);
}

void launch_q4k_norm_multi(const uint8_t* const* w, float* const* y, const int* M, int n, const NormIn& nin,
                           int order, hipStream_t s) {
    const int R = span_rows_per_wave(total_rows(M, n));
    const MultiArgs a = make_multi_args(w, y, M, n, R);
    if (a.first[kMulti] == 0) return;
    if (order == 0) {
        if (R == 1) launch_norm_span<0, 1>(a, nin, s); else launch_norm_span<0, 2>(a, nin, s);
    } else {
        if (R == 1) launch_norm_span<1, 1>(a, nin, s); else launch_norm_span<1, 2>(a, nin, s);
    }
}

template <int ORDER, int NB, int R, int WPB, bool PB>
static int launch_res(const uint8_t* w, int M, const float* x, const ResOut& ro, hipStream_t s) {
    const int g = ((M + R - 1) / R + WPB - 1) / WPB;
    hipLaunchKernelGGL((k_q4k_res_span<ORDER, NB, R, WPB, PB>), dim3(g), dim3(64 * WPB), 0, s, w, M, x, ro);
    return g;
}

// Returns the number of partials written (the grid size).
int launch_q4k_res(const uint8_t* w, int M, const float* x, int K, const ResOut& ro, int order, hipStream_t s) {
    if (K / 256 == 56)
        return order == 0 ? launch_res<0, 56, 1, 8, true>(w, M, x, ro, s) : launch_res<1, 56, 1, 8, true>(w, M, x, ro, s);
    if (span_rows_per_wave(M) == 1)
        return order == 0 ? launch_res<0, 16, 1, 4, false>(w, M, x, ro, s) : launch_res<1, 16, 1, 4, false>(w, M, x, ro, s);
    return order == 0 ? launch_res<0, 16, 2, 4, false>(w, M, x, ro, s) : launch_res<1, 16, 2, 4, false>(w, M, x, ro, s);
}
}  // namespace bpdq
