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
    const uint32_t hd = ld_u16g(blk + 208);
    const float d = f16_ieee(hd);
    const float ds = d * (float)(int8_t)blk[192 + (lane >> 2)];
    f32x4q6 v;
    v.x = ds * (float)((int)(qb & 0xFFu) - 32);
    v.y = ds * (float)((int)((qb >> 8) & 0xFFu) - 32);
    v.z = ds * (float)((int)((qb >> 16) & 0xFFu) - 32);
    v.w = ds * (float)((int)(qb >> 24) - 32);
    // Inf or NaN d (uniform per wave): NaN results take the x86 bits of the
    // reference's (d*sc)*q (numpy float32 for ORDER 0, llama.cpp's C for ORDER 1)
    if (f16_exp31(__builtin_amdgcn_readfirstlane(hd))) {
        v.x = mul_nan_x86(v.x, hd);
        v.y = mul_nan_x86(v.y, hd);
        v.z = mul_nan_x86(v.z, hd);
        v.w = mul_nan_x86(v.w, hd);
    }
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
    const int row0 = (xcd_major(blockIdx.x, gridDim.x) * WPB + wave) * R;
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

// ----------------------------------------------------------------------------
// The same GEMV for K = 4096 (16 super-blocks a row) and 16-byte aligned
// weights, with each wave's two rows read as one contiguous span: 420 aligned
// 16-byte pieces, lane l loading pieces l, l+64, ..., non-temporal, all issued
// before any compute.  Eight super-blocks are 1,680 bytes = 105 whole pieces, so
// before each pass (8 blocks of one row) the wave copies that pass's pieces
// into its own 1,680-byte LDS buffer and the lanes read their operands there in
// k_q6k_q8k_gemv's mapping.  Blocks sit at 210-byte offsets, so odd blocks are
// only 2-byte aligned: words are assembled from aligned dwords with v_alignbit.
// x operands of both passes are loaded (and, in the reference map, regrouped)
// before the span.  Integer sums, c_b and
// the fp32 order are k_q6k_q8k_gemv's, so the bits are the same.
// ----------------------------------------------------------------------------
constexpr int kQ6Pass = 8 * kQ6KBytes;    // 1,680 bytes = 105 pieces
constexpr int kQ6Buf = kQ6Pass + 16;      // tail room for the last aligned dword reads, and the
                                          // slot that takes a lane's out-of-pass piece write

typedef uint32_t q6u32x4 __attribute__((ext_vector_type(4)));

// The 32 q8 values that meet this lane's 32 six-bit values, the bsums of its two
// groups and the block scale.  Reference map: the q8 bytes regrouped to match
// the nibble and 2-bit fields as they sit in ql and qh (see q6k_lane_isum_lds):
// xs[2m], xs[2m+1] = the even / odd elements of 8m..8m+7 (m < 4), and
// xs[8+4n+k] = elements 16n+k, 16n+4+k, 16n+8+k, 16n+12+k (n < 2, k < 4).
// GGUF map: xs[0..7] = elements e0.. and e1.. as loaded.
template <int ORDER>
struct Q6X {
    uint32_t xs[ORDER == 0 ? 16 : 8];
    int bs0, bs1;
    float dy;
};

// The Q8_K bytes a lane needs for super-block xb (load_q6x's loads).
struct Q6XRaw {
    uint32_t raw[8];
    int16_t b0, b1;
    float dy;
};

template <int ORDER>
__device__ __forceinline__ void q6x_fields(int c, int& g0, int& g1, int& e0, int& e1) {
    if (ORDER == 0) {
        g0 = 2 * c;
        e0 = 32 * c;
        e1 = e0 + 16;
    } else {
        const int h = c >> 2, p = c & 3;
        g0 = 8 * h + p;
        e0 = 128 * h + 16 * p;
        e1 = e0 + 64;
    }
    g1 = ORDER == 0 ? g0 + 1 : g0 + 4;
}

template <int ORDER>
__device__ __forceinline__ Q6XRaw q6x_load_raw(const uint8_t* __restrict__ xb, int c) {
    Q6XRaw r;
    int g0, g1, e0, e1;
    q6x_fields<ORDER>(c, g0, g1, e0, e1);
    __builtin_memcpy(&r.dy, xb, 4);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        r.raw[k] = ld_u32(xb + 4 + e0 + 4 * k);
        r.raw[4 + k] = ld_u32(xb + 4 + e1 + 4 * k);
    }
    __builtin_memcpy(&r.b0, xb + 260 + 2 * g0, 2);
    __builtin_memcpy(&r.b1, xb + 260 + 2 * g1, 2);
    return r;
}

template <int ORDER>
__device__ __forceinline__ Q6X<ORDER> q6x_regroup(const Q6XRaw& r) {
    Q6X<ORDER> o;
    o.dy = r.dy;
    const uint32_t* raw = r.raw;
    if constexpr (ORDER == 0) {
#pragma unroll
        for (int m = 0; m < 4; m++) {
            o.xs[2 * m] = __builtin_amdgcn_perm(raw[2 * m + 1], raw[2 * m], 0x06040200u);      // even elements
            o.xs[2 * m + 1] = __builtin_amdgcn_perm(raw[2 * m + 1], raw[2 * m], 0x07050301u);  // odd elements
        }
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t sel = (uint32_t)k | ((uint32_t)(k + 4) << 8);  // byte k of S1, byte k of S0
                const uint32_t t1 = __builtin_amdgcn_perm(raw[4 * n + 1], raw[4 * n], sel);
                const uint32_t t2 = __builtin_amdgcn_perm(raw[4 * n + 3], raw[4 * n + 2], sel);
                o.xs[8 + 4 * n + k] = __builtin_amdgcn_perm(t2, t1, 0x05040100u);
            }
    } else {
#pragma unroll
        for (int k = 0; k < 8; k++) o.xs[k] = raw[k];
    }
    o.bs0 = r.b0;
    o.bs1 = r.b1;
    return o;
}

template <int ORDER>
__device__ __forceinline__ Q6X<ORDER> load_q6x(const uint8_t* __restrict__ xb, int c) {
    return q6x_regroup<ORDER>(q6x_load_raw<ORDER>(xb, c));
}

// N consecutive words starting at LDS address p, p % 4 in {0, 2}.  The aligned
// base is p minus its misalignment (pointer arithmetic: a pointer rebuilt from
// an integer loses the LDS address space, and its reads become flat loads that
// wait on every outstanding global load too).
template <int N>
__device__ __forceinline__ void lds_words_a2(const uint8_t* p, uint32_t (&out)[N]) {
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;
    const uint32_t* base = static_cast<const uint32_t*>(__builtin_assume_aligned(p - mis, 4));
    const uint32_t sh = 8u * mis;
    uint32_t d[N + 1];
#pragma unroll
    for (int i = 0; i <= N; i++) d[i] = base[i];
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbit(d[i + 1], d[i], sh);
}

template <int ORDER>
__device__ __forceinline__ int q6k_lane_isum_lds(const uint8_t* blk, const Q6X<ORDER>& x, int c) {
    int S0 = 0, S1 = 0, g0, g1;
    if constexpr (ORDER == 0) {
        // elements 32c+e: ql byte e/2 holds e (low nibble) and e+1 (high), qh byte e/4
        // holds bits 2(e%4).. of e.  The sum over a group is exact in any order, so
        // dot the fields where they sit against the regrouped x:
        //   S = sum_m [low nibbles of ql dword m . even x] + [high nibbles . odd x]
        //     + 16 * sum_{n,k} [bits 2k..2k+1 of the qh dword n bytes . xs[8+4n+k]]
        g0 = 2 * c;
        g1 = 2 * c + 1;
        uint32_t qlw[4], qhw[2];
        lds_words_a2<4>(blk + 16 * c, qlw);
        lds_words_a2<2>(blk + 128 + 8 * c, qhw);
        int H0 = 0, H1 = 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            int& S = m < 2 ? S0 : S1;
            S = sdot4(qlw[m] & 0x0F0F0F0Fu, x.xs[2 * m], S);
            S = sdot4((qlw[m] >> 4) & 0x0F0F0F0Fu, x.xs[2 * m + 1], S);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            H0 = sdot4((qhw[0] >> (2 * k)) & 0x03030303u, x.xs[8 + k], H0);
            H1 = sdot4((qhw[1] >> (2 * k)) & 0x03030303u, x.xs[12 + k], H1);
        }
        S0 += 16 * H0;
        S1 += 16 * H1;
    } else {
        const int h = c >> 2, p = c & 3, sh = 2 * (p >> 1);
        g0 = 8 * h + p;
        g1 = g0 + 4;
        uint32_t qlw[4], qhw[4];
        lds_words_a2<4>(blk + 64 * h + 16 * p, qlw);
        lds_words_a2<4>(blk + 128 + 32 * h + 16 * (p & 1), qhw);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo = q6_bytes(qlw[k], qhw[k] >> sh);
            const uint32_t hi = q6_bytes(qlw[k] >> 4, qhw[k] >> (sh + 4));
            S0 = sdot4(lo, x.xs[k], S0);
            S1 = sdot4(hi, x.xs[4 + k], S1);
        }
    }
    const int sc0 = (int8_t)blk[192 + g0], sc1 = (int8_t)blk[192 + g1];
    return sc0 * (S0 - 32 * x.bs0) + sc1 * (S1 - 32 * x.bs1);
}

template <int ORDER, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q6k_q8k_gemv_span(const uint8_t* __restrict__ w,
                                                               const uint8_t* __restrict__ xq, float* __restrict__ y,
                                                               int M) {
    constexpr int NB = 16, R = 2, NT = NB / 8;
    constexpr int kPieces = R * NB * kQ6KBytes / 16;  // 420
    constexpr int kLoads = (kPieces + 63) / 64;       // 7
    __shared__ __align__(16) uint8_t bufs[WPB][kQ6Buf];
    const int lane = threadIdx.x & 63;
    const int q = lane >> 3, c = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (xcd_major(blockIdx.x, gridDim.x) * WPB + wave) * R;
    if (row0 >= M) return;
    Q6X<ORDER> x[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) x[t] = load_q6x<ORDER>(xq + (int64_t)(8 * t + q) * kQ8KBytes, c);
    // rows past M repeat the last piece of row M-1 (their results are not stored)
    const uint8_t* span = w + (int64_t)row0 * (NB * kQ6KBytes);
    const int np = min(R, M - row0) * NB * kQ6KBytes / 16;
    q6u32x4 v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
        const uint32_t p = (uint32_t)min(lane + 64 * u, np - 1);
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const q6u32x4*>(span + 16u * p));
    }
    uint8_t* buf = bufs[wave];
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            // the pass's 105 pieces, in order (the previous pass's reads were consumed
            // before these writes)
            const int p0 = (r * NB + 8 * t) * kQ6KBytes / 16, n = kQ6Pass / 16;
#pragma unroll
            for (int u = 0; u < kLoads; u++) {
                if (64 * u + 63 < p0 || 64 * u >= p0 + n) continue;
                // pieces outside the pass go to the spare slot n: no branch around
                // the write, so the compiler's load waits stay per load
                const int k = lane + 64 * u - p0;
                *reinterpret_cast<q6u32x4*>(buf + 16 * (k >= 0 && k < n ? k : n)) = v[u];
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            const uint8_t* blk = buf + q * kQ6KBytes;
            int isum = q6k_lane_isum_lds<ORDER>(blk, x[t], c);
            isum = sum8_i(isum);
            uint16_t dh;
            __builtin_memcpy(&dh, blk + 208, 2);
            const float dd = f16_ieee(dh) * x[t].dy;
            float acc = s[r] + dd * (float)isum;
            // this pass's arithmetic is done before the next pass's LDS writes (which
            // wait for their loads), not hoisted below them
            asm volatile("" : "+v"(acc) : : "memory");
            s[r] = acc;
        }
    }
    // k_q6k_q8k_gemv's combine
#pragma unroll
    for (int r = 0; r < R; r++) {
        float tv = s[r];
        tv = tv + dpp_f<0x140>(tv);
        const float p01 = readlane_f(tv, 0), p23 = readlane_f(tv, 16);
        const float p45 = readlane_f(tv, 32), p67 = readlane_f(tv, 48);
        if (lane == 0 && row0 + r < M) y[row0 + r] = (p01 + p23) + (p45 + p67);
    }
}

// K = 14336 (56 super-blocks): one row per wave (735 pieces, 12 loads per lane)
// in the same 8-block passes.  The x operands of 7 passes would not fit the
// registers, so the workgroup first stages them in LDS, already in the lanes'
// form: thread t < 448 loads the Q8_K bytes of (super-block t/8, lane group t%8)
// before the span loads are issued, regroups them after (the perm work of
// load_q6x, done once per workgroup instead of once per wave and pass) and
// stores one 80-byte record; one barrier; each pass reads its record with
// aligned 16-byte LDS reads.
template <int ORDER, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_q6k_q8k_gemv_span_long(const uint8_t* __restrict__ w,
                                                                    const uint8_t* __restrict__ xq,
                                                                    float* __restrict__ y, int M) {
    constexpr int NB = 56, NT = NB / 8;
    constexpr int kPieces = NB * kQ6KBytes / 16;  // 735
    constexpr int kLoads = (kPieces + 63) / 64;   // 12
    constexpr int XR = NB * 8;                    // x records: (super-block, lane group)
    constexpr int kRec = 20;                      // dwords: xs[16], bs0, bs1, dy, pad
    static_assert(XR <= 64 * WPB, "one record per thread");
    __shared__ __align__(16) uint8_t bufs[WPB][kQ6Buf];
    __shared__ __align__(16) uint32_t xrec[XR * kRec];
    const int tid = threadIdx.x, lane = tid & 63;
    const int q = lane >> 3, c = lane & 7;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = xcd_major(blockIdx.x, gridDim.x) * WPB + wave;
    const bool has = row < M;
    // threads past the last record load record XR-1's bytes again (not stored)
    const int rt = min(tid, XR - 1);
    const Q6XRaw xr = q6x_load_raw<ORDER>(xq + (int64_t)(rt >> 3) * kQ8KBytes, rt & 7);
    // waves past the last row read row M-1 (nothing is stored for them)
    const uint8_t* span = w + (int64_t)(has ? row : M - 1) * (NB * kQ6KBytes);
    q6u32x4 v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
        const uint32_t p = (uint32_t)min(lane + 64 * u, kPieces - 1);
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const q6u32x4*>(span + 16u * p));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < XR) {
        const Q6X<ORDER> xo = q6x_regroup<ORDER>(xr);
        uint32_t* rec = xrec + tid * kRec;
#pragma unroll
        for (int k2 = 0; k2 < (ORDER == 0 ? 16 : 8); k2++) rec[k2] = xo.xs[k2];
        rec[16] = (uint32_t)xo.bs0;
        rec[17] = (uint32_t)xo.bs1;
        rec[18] = __float_as_uint(xo.dy);
    }
    __syncthreads();
    // waves past the last row run on (no early return: the compiler would sink the
    // span loads below it, after the x copy and the barrier) and store nothing
    uint8_t* buf = bufs[wave];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int p0 = 8 * t * kQ6KBytes / 16, n = kQ6Pass / 16;
#pragma unroll
        for (int u = 0; u < kLoads; u++) {
            if (64 * u + 63 < p0 || 64 * u >= p0 + n) continue;
            const int k = lane + 64 * u - p0;  // outside the pass: the spare slot n
            *reinterpret_cast<q6u32x4*>(buf + 16 * (k >= 0 && k < n ? k : n)) = v[u];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        Q6X<ORDER> x;
        {
            const uint32_t* rec = xrec + ((8 * t + q) * 8 + c) * kRec;
#pragma unroll
            for (int k2 = 0; k2 < (ORDER == 0 ? 16 : 8); k2++) x.xs[k2] = rec[k2];
            x.bs0 = (int)rec[16];
            x.bs1 = (int)rec[17];
            x.dy = __uint_as_float(rec[18]);
        }
        const uint8_t* blk = buf + q * kQ6KBytes;
        int isum = q6k_lane_isum_lds<ORDER>(blk, x, c);
        isum = sum8_i(isum);
        uint16_t dh;
        __builtin_memcpy(&dh, blk + 208, 2);
        s = s + (f16_ieee(dh) * x.dy) * (float)isum;
        asm volatile("" : "+v"(s) : : "memory");  // as in k_q6k_q8k_gemv_span
    }
    s = s + dpp_f<0x140>(s);
    const float p01 = readlane_f(s, 0), p23 = readlane_f(s, 16);
    const float p45 = readlane_f(s, 32), p67 = readlane_f(s, 48);
    if (lane == 0 && has) y[row] = (p01 + p23) + (p45 + p67);
}

void launch_qmatmul_q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, hipStream_t s) {
    if (K == 14336 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
        constexpr int WPB = 8;
        const dim3 grid((M + WPB - 1) / WPB);
        if (order == 0)
            hipLaunchKernelGGL((k_q6k_q8k_gemv_span_long<0, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M);
        else
            hipLaunchKernelGGL((k_q6k_q8k_gemv_span_long<1, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M);
        return;
    }
    if (K == 4096 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
        constexpr int WPB = 4;
        const int waves = (M + 1) / 2;
        const dim3 grid((waves + WPB - 1) / WPB);
        if (order == 0)
            hipLaunchKernelGGL((k_q6k_q8k_gemv_span<0, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M);
        else
            hipLaunchKernelGGL((k_q6k_q8k_gemv_span<1, WPB>), grid, dim3(64 * WPB), 0, s, w, xq, y, M);
        return;
    }
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
