// q6k.hip — Q6_K super-block kernels for gfx950.
//
//   k_dequant_q6k<ORDER>        Q6_K -> fp32
//   k_q6k_q8k_gemv<ORDER>       Q6_K x Q8_K GEMV, exact integer group sums + fixed fp32 tree
//
// Q6_K block, 210 B per 256 elements: ql[128] (low 4 bits), qh[64] (high 2 bits),
// sc[16] (int8, element e uses sc[e/16]), d (f16 at byte 208); q = low | high<<4, minus 32.
// Element maps:
//   ORDER 0 (inference/llamatov_helpers.py:161-179): element 2i takes the low nibble
//            of ql[i], 2i+1 the high nibble; element 4j+k takes bits 2k..2k+1 of qh[j].
//   ORDER 1 (GGUF / llama.cpp dequantize_row_q6_K): in half h (ql += 64h, qh += 32h),
//            for l < 32: element l = ql[l] low + qh[l] bits 0-1, l+32 = ql[l+32] low +
//            bits 2-3, l+64 = ql[l] high + bits 4-5, l+96 = ql[l+32] high + bits 6-7.
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

constexpr int kQ6KBytes = 210;

__device__ __forceinline__ uint32_t ld_u16g(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Four 6-bit values (0..63, i.e. q + 32) as bytes: low nibbles in bits 0-3 of
// each byte of `lo4`, the 2-bit high parts in bits 0-1 of each byte of `hi2`.
__device__ __forceinline__ uint32_t q6_bytes(uint32_t lo4, uint32_t hi2) {
    return (lo4 & 0x0F0F0F0Fu) | ((hi2 & 0x03030303u) << 4);
}

// ORDER 0 helpers: the 4 elements 4j..4j+3 take the nibbles of ql[2j] (lo, hi)
// and ql[2j+1] (lo, hi), and bits (0,1) (2,3) (4,5) (6,7) of qh[j].
__device__ __forceinline__ uint32_t spread_nibbles(uint32_t two_bytes) {
    // bytes [b0, b0, b1, b1]; then byte 0 keeps b0 low, byte 1 b0 high, ...
    const uint32_t dup = __builtin_amdgcn_perm(0u, two_bytes, 0x01010000u);
    return (dup & 0x000F000Fu) | ((dup >> 4) & 0x0F000F00u);
}
__device__ __forceinline__ uint32_t spread_pairs(uint32_t byte) {
    // byte k of the result holds bits 2k..2k+1 of `byte` in its low two bits
    return (byte & 0x3u) | ((byte << 6) & 0x300u) | ((byte << 12) & 0x30000u) | ((byte << 18) & 0x3000000u);
}

// ----------------------------------------------------------------------------
// Dequant.  One wave per block; lane l writes elements 4l..4l+3 as one 16-byte
// non-temporal store.  y = (d * sc) * q: d*sc is exact (11 x 8 bits), so this
// is RN(d*sc*q), the reference's float32 numpy value.
// ----------------------------------------------------------------------------
typedef float f32x4q6 __attribute__((ext_vector_type(4)));

template <int ORDER>
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t* __restrict__ q, float* __restrict__ out,
                                                     int n_blocks) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= n_blocks) return;
    const uint8_t* blk = q + b * kQ6KBytes;
    uint32_t qb;  // the four values q + 32 as bytes
    if (ORDER == 0) {
        const uint32_t ql2 = ld_u16g(blk + 2 * lane);
        const uint32_t qh = blk[128 + lane];
        qb = q6_bytes(spread_nibbles(ql2), spread_pairs(qh));
    } else {
        const int e0 = 4 * lane, h = e0 >> 7, r = e0 & 127, quarter = r >> 5, idx = r & 31;
        const uint32_t ql4 = ld_u32(blk + 64 * h + 32 * (quarter & 1) + idx);
        const uint32_t qh4 = ld_u32(blk + 128 + 32 * h + idx);
        qb = q6_bytes(ql4 >> (4 * (quarter >> 1)), qh4 >> (2 * quarter));
    }
    const float d = f16_ieee(ld_u16g(blk + 208));
    const float ds = d * (float)(int8_t)blk[192 + (lane >> 2)];
    f32x4q6 v;
    v.x = ds * (float)((int)(qb & 0xFFu) - 32);
    v.y = ds * (float)((int)((qb >> 8) & 0xFFu) - 32);
    v.z = ds * (float)((int)((qb >> 16) & 0xFFu) - 32);
    v.w = ds * (float)((int)(qb >> 24) - 32);
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4q6*>(out + b * 256 + 4 * lane));
}

void launch_dequant_q6k(const uint8_t* q, float* out, int n_blocks, int order, hipStream_t s) {
    const dim3 grid((unsigned)(((int64_t)n_blocks + 3) / 4));
    if (order == 0)
        hipLaunchKernelGGL(k_dequant_q6k<0>, grid, dim3(256), 0, s, q, out, n_blocks);
    else
        hipLaunchKernelGGL(k_dequant_q6k<1>, grid, dim3(256), 0, s, q, out, n_blocks);
}

// ----------------------------------------------------------------------------
// Q6_K x Q8_K GEMV.  Lane (q = lane/8, c = lane%8) owns 32 elements of
// super-block 8t+q, two scale groups:
//   ORDER 0: elements 32c..32c+31 = ql[16c..16c+15], qh[8c..8c+7], groups 2c, 2c+1;
//   ORDER 1: h = c/4, p = c%4: ql[64h+16p..+15], qh[32h+16(p%2)..+15]; low nibbles
//            are elements 128h+16p+i (group 8h+p, qh shift 2(p/2)), high nibbles
//            elements 128h+16p+64+i (group 8h+p+4, qh shift 2(p/2)+4).
// S_g = dot(q+32, x) - 32*bsum_g is exact; I_b = sum_g sc_g*S_g over the 8
// lanes (exact); c_b = RN(RN(d*dy) * float(I_b)); then the slot sums and tree
// of the Q4_K x Q8_K GEMV, so the fp32 order is the one restated in the oracle.
// ----------------------------------------------------------------------------
template <int ORDER>
__device__ __forceinline__ int q6k_lane_isum(const uint8_t* __restrict__ blk, const uint8_t* __restrict__ xb, int c) {
    int S0 = 0, S1 = 0, g0, g1;
    if (ORDER == 0) {
        g0 = 2 * c;
        g1 = 2 * c + 1;
        const uint4 ql = *reinterpret_cast<const uint4*>(blk + 16 * c);  // 32 nibbles
        const uint2 qh = *reinterpret_cast<const uint2*>(blk + 128 + 8 * c);
        const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t qhw[2] = {qh.x, qh.y};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t two = (qlw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
            const uint32_t hb = (qhw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            const uint32_t qv = q6_bytes(spread_nibbles(two), spread_pairs(hb));
            const uint32_t xv = ld_u32(xb + 4 + 32 * c + 4 * j);
            if (j < 4)
                S0 = sdot4(qv, xv, S0);
            else
                S1 = sdot4(qv, xv, S1);
        }
    } else {
        const int h = c >> 2, p = c & 3, sh = 2 * (p >> 1);
        g0 = 8 * h + p;
        g1 = g0 + 4;
        const uint4 ql = *reinterpret_cast<const uint4*>(blk + 64 * h + 16 * p);
        const uint4 qh = *reinterpret_cast<const uint4*>(blk + 128 + 32 * h + 16 * (p & 1));
        const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        const int e0 = 128 * h + 16 * p;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo = q6_bytes(qlw[k], qhw[k] >> sh);
            const uint32_t hi = q6_bytes(qlw[k] >> 4, qhw[k] >> (sh + 4));
            S0 = sdot4(lo, ld_u32(xb + 4 + e0 + 4 * k), S0);
            S1 = sdot4(hi, ld_u32(xb + 4 + e0 + 64 + 4 * k), S1);
        }
    }
    int16_t bs0, bs1;
    __builtin_memcpy(&bs0, xb + 260 + 2 * g0, 2);
    __builtin_memcpy(&bs1, xb + 260 + 2 * g1, 2);
    const int sc0 = (int8_t)blk[192 + g0], sc1 = (int8_t)blk[192 + g1];
    return sc0 * (S0 - 32 * (int)bs0) + sc1 * (S1 - 32 * (int)bs1);
}

template <int ORDER, int R, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q6k_q8k_gemv(const uint8_t* __restrict__ w,
                                                           const uint8_t* __restrict__ xq, float* __restrict__ y,
                                                           int M, int nb) {
    const int lane = threadIdx.x & 63;
    const int q = lane >> 3, c = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (blockIdx.x * WPB + wave) * R;
    if (row0 >= M) return;
    const int64_t row_bytes = (int64_t)nb * kQ6KBytes;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;
    for (int t = 0; t * 8 < nb; t++) {
        const int b = 8 * t + q;
        const bool valid = b < nb;
        const int bb = valid ? b : nb - 1;
        const uint8_t* xb = xq + (int64_t)bb * kQ8KBytes;
        float dy;
        __builtin_memcpy(&dy, xb, 4);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t* blk = w + (int64_t)min(row0 + r, M - 1) * row_bytes + (int64_t)bb * kQ6KBytes;
            int isum = q6k_lane_isum<ORDER>(blk, xb, c);
            isum = sum8_i(isum);
            const float dd = f16_ieee(ld_u16g(blk + 208)) * dy;
            const float cb = dd * (float)isum;
            if (valid) s[r] = s[r] + cb;
        }
    }
    // slot q lives in lanes 8q..8q+7: row_mirror pairs slots q and q^1, then the
    // four pair sums are lanes 0, 16, 32, 48
#pragma unroll
    for (int r = 0; r < R; r++) {
        float v = s[r];
        v = v + dpp_f<0x140>(v);
        const float p01 = readlane_f(v, 0), p23 = readlane_f(v, 16);
        const float p45 = readlane_f(v, 32), p67 = readlane_f(v, 48);
        if (lane == 0 && row0 + r < M) y[row0 + r] = (p01 + p23) + (p45 + p67);
    }
}

void launch_qmatmul_q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s) {
    constexpr int R = 2, WPB = 4;
    const int nb = K / 256;
    const int waves = (M + R - 1) / R;
    const dim3 grid((waves + WPB - 1) / WPB);
    if (order == 0)
        hipLaunchKernelGGL((k_q6k_q8k_gemv<0, R, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M, nb);
    else
        hipLaunchKernelGGL((k_q6k_q8k_gemv<1, R, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M, nb);
}

}  // namespace bpdq
