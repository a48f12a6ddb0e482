// bpdq_device.h — device helpers shared by the gfx950 kernels.
//
// All kernels are compiled with -ffp-contract=off: every fp32 expression is the
// sequence of IEEE operations written, and an FMA appears only where fmaf() is
// called explicitly (and only where it is provably equal to the unfused form).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bpdq {

constexpr int kQ4KBytes = 144;   // {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}
constexpr int kQ8KBytes = 292;   // {f32 d, i8 qs[256], i16 bsums[16]}
constexpr int kQ80Bytes = 34;    // {f16 d, i8 qs[32]}

// IEEE binary16 -> binary32 (v_cvt_f32_f16): exact for every finite input and
// for +/-0 and +/-Inf.  NaN stays NaN.
__device__ __forceinline__ float f16_ieee(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// The decode of /root/reference/bench/bench_dequant_gpu_h2h.cu:14-19: both
// zeros -> +0.0, exponent 31 (Inf or NaN) -> +/-Inf, all else exact.
__device__ __forceinline__ float f16_h2h(uint32_t h) {
    h &= 0xFFFFu;
    if ((h & 0x7FFFu) == 0) return 0.0f;
    if ((h & 0x7C00u) == 0x7C00u) return (h & 0x8000u) ? -__builtin_inff() : __builtin_inff();
    return f16_ieee(h);
}

// ---- NaN bits of the reference builds ---------------------------------------
// The reference's C runs on x86: an SSE operation gives a NaN operand back
// quieted (the first operand's when both are NaN) and the default NaN
// 0xFFC00000 for an invalid operation (Inf*0, Inf-Inf).  Its CUDA kernels run on
// NVIDIA GPUs, whose fp32 operations return the canonical NaN 0x7FFFFFFF.  The
// kernels below compute as usual and, only where the result is NaN (which the
// IEEE rules make NaN on every machine alike), select those bits.
constexpr uint32_t kX86NaN = 0xFFC00000u;
constexpr uint32_t kCudaNaN = 0x7FFFFFFFu;

__device__ __forceinline__ bool f16_is_nan(uint32_t h) { return (h & 0x7FFFu) > 0x7C00u; }
__device__ __forceinline__ bool f16_is_inf(uint32_t h) { return (h & 0x7FFFu) == 0x7C00u; }
__device__ __forceinline__ bool f16_exp31(uint32_t h) { return (h & 0x7C00u) == 0x7C00u; }

// An f16 NaN as the magic-number decode of /root/reference/bench/bpd_cpu.c:3928-3958
// leaves it after a multiply: sign, the payload shifted up, the quiet bit set.
__device__ __forceinline__ float f16_nan_x86(uint32_t h) {
    return __uint_as_float(((h & 0x8000u) << 16) | 0x7FC00000u | ((h & 0x3FFu) << 13));
}

// x86 result bits of a binary operation r = first OP second whose result is NaN.
__device__ __forceinline__ float x86_nan_of(float first, float second) {
    if (__builtin_isnan(first)) return __uint_as_float(__float_as_uint(first) | 0x400000u);
    if (__builtin_isnan(second)) return __uint_as_float(__float_as_uint(second) | 0x400000u);
    return __uint_as_float(kX86NaN);
}

// Bits of a NaN Q4_K element y = RN(d*sc*q - dmin*m) as the reference computes it
// on x86 (/root/reference/bench/bpd_quant.c:25-38,64-71): half_to_float turns an
// f16 NaN into +/-0x7FC00000 without payload; d*sc and then *q propagate d's NaN
// or make the default NaN from Inf*0; the subtraction keeps the left NaN, else
// dmin*m's.  So y's NaN is positive only when it comes from a positive NaN d, or,
// with no NaN on the left, from a positive NaN dmin.  hd, hm: the f16 bits of d
// and dmin.  Returns y unchanged when it is not NaN.
__device__ __forceinline__ float q4k_bpd_nan(float y, uint32_t hd, uint32_t hm, int sc, uint32_t q) {
    if (!__builtin_isnan(y)) return y;
    bool pos;
    if (f16_is_nan(hd)) pos = (hd & 0x8000u) == 0;
    else if (f16_is_inf(hd) && (sc == 0 || q == 0)) pos = false;
    else pos = f16_is_nan(hm) && (hm & 0x8000u) == 0;
    return __uint_as_float(pos ? 0x7FC00000u : kX86NaN);
}

// A NaN product d*c (c an integer-valued fp32, d decoded by the magic-number
// form): d's NaN quieted, else (Inf*0) the default NaN.  Q8_0 dequant
// (/root/reference/bench/bpd_cpu.c:3960-3973) and Q6_K dequant.
__device__ __forceinline__ float mul_nan_x86(float y, uint32_t hd) {
    if (!__builtin_isnan(y)) return y;
    return f16_is_nan(hd) ? f16_nan_x86(hd) : __uint_as_float(kX86NaN);
}

// 6-bit scale and min of sub-block j from the 12 scale bytes held in three
// dwords s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11
// (layout of /root/reference/bench/bpd_quant.c:56-62):
//   j < 4 : sc = s[j] & 63,                         m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | ((s[j-4] >> 6) << 4), m = (s[j+4] >> 4) | ((s[j] >> 6) << 4)
// Both halves are computed and selected, so a lane-varying j never becomes a branch.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc, int& m) {
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t a = s0 >> sh, b = s1 >> sh, h = s2 >> sh;
    const uint32_t sc_hi = (h & 15u) | ((a >> 2) & 0x30u);
    const uint32_t m_hi = ((h >> 4) & 15u) | ((b >> 2) & 0x30u);
    sc = (int)(j < 4 ? (a & 63u) : sc_hi);
    m = (int)(j < 4 ? (b & 63u) : m_hi);
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations complete, then
// s_barrier.  Unlike __syncthreads() it does not wait for the wave's outstanding
// global loads, so a register prefetch stays in flight across it.  Only for
// kernels whose waves exchange data through LDS alone.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Nonzero when some byte of v is 0x80 (-128).
__device__ __forceinline__ uint32_t has_m128(uint32_t v) {
    const uint32_t t = v ^ 0x80808080u;
    return (t - 0x01010101u) & ~t & 0x80808080u;
}

// The AVX1 builds' int8 products: _mm_maddubs_epi16(_mm_sign_epi8(w, w),
// _mm_sign_epi8(a, w)) and _mm_madd_epi16 with ones, over the 4 bytes of one
// dword: |w| read as an unsigned byte (128 for -128), a*sign(w) wrapping (-(-128)
// is -128), each pair's sum saturated to int16, the two pairs added.  Equal to
// the exact dot whenever no byte of a is -128 against a negative w.
__device__ __forceinline__ int ssse3_quad_inl(uint32_t w, uint32_t a) {
    int total = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        int t = 0;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int wi = (int8_t)(w >> (16 * h + 8 * u)), ai = (int8_t)(a >> (16 * h + 8 * u));
            const int uw = wi < 0 ? -wi : wi;
            const int sa = wi < 0 ? (int)(int8_t)(uint8_t)(-ai) : (wi == 0 ? 0 : ai);
            t += uw * sa;
        }
        total += t > 32767 ? 32767 : (t < -32768 ? -32768 : t);
    }
    return total;
}

// Cross-lane moves inside a wave64.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// v_permlane32_swap: afterwards a's lanes 32-63 hold b's old lanes 0-31 and b's
// lanes 0-31 hold a's old lanes 32-63 (the other halves are unchanged).
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r.x;
    b = r.y;
}
__device__ __forceinline__ float xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }
__device__ __forceinline__ int xor_i(int v, int mask) { return __shfl_xor(v, mask, 64); }

// Sum of an int over each aligned group of 8 lanes (exact; order irrelevant).
__device__ __forceinline__ int sum8_i(int v) {
    v += dpp_i<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_i<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_i<0x141>(v);  // row_half_mirror: lane i <-> 7-i inside each 8
    return v;
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

__device__ __forceinline__ uint4 ld_u128(const uint8_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// The quantizers' multiplier id = 127/amax (0 when amax is 0), made 0 where it
// overflows to +Inf (amax < 127/FLT_MAX).  The reference's (int8_t)rintf(x*id)
// (/root/reference/bench/bpd_cpu.c:4133) runs on x86 as cvttss2si to int32 (0x80000000
// for NaN and out-of-range values) and keeps the low byte: every non-finite x*id
// gives quant 0.  v_cvt_i32_f32 gives 0 for NaN and 0x80000000 for -Inf too, but
// saturates +Inf to 0x7FFFFFFF (byte 0xFF); with a finite id, x*id is never +Inf
// (|x| <= amax, and x = Inf makes amax = Inf and id = 0: NaN), and with id = 0 in
// place of +Inf every quant of the block is 0 or NaN -> 0, as on x86.  So the plain
// conversion of rint(x*q8_id(amax)) gives the reference's bytes for every input.
__device__ __forceinline__ float q8_id(float amax) {
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    return __builtin_isinf(id) ? 0.0f : id;
}

// |v| for the quantizers' amax: the reference's scalar loop (`if (av > max)`,
// max starting at 0) never takes a NaN, so a NaN element counts as 0 and a block
// of NaNs keeps amax = 0.  maxNum(|v|, 0) is |v|, or 0 for a NaN (the compiler
// quiets a signalling NaN before v_max_f32), so the reduction never meets a NaN.
__device__ __forceinline__ float abs_no_nan(float v) { return fmaxf(fabsf(v), 0.0f); }

// Q8_0 quantization of one 32-element block held by 32 consecutive lanes of a
// wave (lane = element e, all 32 active), as bpd_quant_q8_0_cpu
// (/root/reference/bench/bpd_cpu.c:4106-4136) computes it: amax is exact in any
// order (NaN never wins, as with its `av > max` test: abs_no_nan); d = RN(amax/127) is stored
// as an RNE binary16 (v_cvt_f16_f32); id = RN(127/amax); q = rint(RN(v*id)).
__device__ __forceinline__ void q8_0_lane_store(float v, uint8_t* __restrict__ yb, int e) {
    float amax = abs_no_nan(v);
#pragma unroll
    for (int mask = 1; mask < 32; mask <<= 1) amax = fmaxf(amax, xor_f(amax, mask));
    const float d = amax / 127.0f;
    const float id = q8_id(amax);
    yb[2 + e] = (uint8_t)(int8_t)(int)__builtin_rintf(v * id);
    if (e == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);
        yb[0] = (uint8_t)(h & 0xFF);
        yb[1] = (uint8_t)(h >> 8);
    }
}

// The same bytes from 8 consecutive lanes holding 4 elements each (lane g of
// the aligned group holds elements 4g..4g+3).  yb is a 34-byte record, so only
// 2-byte aligned: the quants go out as two 16-bit stores per lane.
__device__ __forceinline__ void q8_0_quad_store(float4 v, uint8_t* __restrict__ yb, int g) {
    float amax = fmaxf(fmaxf(abs_no_nan(v.x), abs_no_nan(v.y)), fmaxf(abs_no_nan(v.z), abs_no_nan(v.w)));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror: the other quad of the 8
    const float d = amax / 127.0f;
    const float id = q8_id(amax);
    const uint32_t q0 = (uint32_t)(int)__builtin_rintf(v.x * id) & 0xFFu;
    const uint32_t q1 = (uint32_t)(int)__builtin_rintf(v.y * id) & 0xFFu;
    const uint32_t q2 = (uint32_t)(int)__builtin_rintf(v.z * id) & 0xFFu;
    const uint32_t q3 = (uint32_t)(int)__builtin_rintf(v.w * id) & 0xFFu;
    uint16_t* p = reinterpret_cast<uint16_t*>(yb + 2 + 4 * g);
    p[0] = (uint16_t)(q0 | (q1 << 8));
    p[1] = (uint16_t)(q2 | (q3 << 8));
    if (g == 0) *reinterpret_cast<uint16_t*>(yb) = __builtin_bit_cast(uint16_t, (_Float16)d);
}

// The same bytes from 16 consecutive lanes holding 2 elements each (lane g of the
// aligned 16-lane row holds elements 2g, 2g+1); two bytes per lane.
__device__ __forceinline__ void q8_0_pair_store(float2 v, uint8_t* __restrict__ yb, int g) {
    float amax = fmaxf(abs_no_nan(v.x), abs_no_nan(v.y));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror: the other quad of the 8
    amax = fmaxf(amax, dpp_f<0x140>(amax));  // row_mirror: the other 8 of the row
    const float d = amax / 127.0f;
    const float id = q8_id(amax);
    const uint32_t q0 = (uint32_t)(int)__builtin_rintf(v.x * id) & 0xFFu;
    const uint32_t q1 = (uint32_t)(int)__builtin_rintf(v.y * id) & 0xFFu;
    *reinterpret_cast<uint16_t*>(yb + 2 + 2 * g) = (uint16_t)(q0 | (q1 << 8));
    if (g == 0) *reinterpret_cast<uint16_t*>(yb) = __builtin_bit_cast(uint16_t, (_Float16)d);
}

// Workgroup b of a grid of G workgroups as numbered for row order.  The
// hardware hands workgroups to the 8 XCDs round robin (b % 8), each XCD with
// its own L2: XCD-major numbering gives each XCD one contiguous range of rows,
// so each 128-byte line of outputs (rows of several workgroups) is written from
// one L2 instead of four.  When G is not a multiple of 8, b itself.
__device__ __forceinline__ int xcd_major(int b, int G) {
    return (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
}

// RMSNorm's scale 1 / sqrtf(mean + eps) (bpd_rmsnorm_llama_cpu,
// bench/bpd_cpu.c:4959-4986: a sequential binary64 sum of (double)x^2, mean =
// (float)(sum / n)) from S, the binary64 sum of the same n squares in another
// order.  Any order of n non-negative terms is within (n - 1) 2^-53 S of the
// exact sum, as is the sequential one, so when (S - E)/n and (S + E)/n, E =
// 4 n 2^-53 S, round to the same float, rounding monotonicity pins the
// reference's mean to it; otherwise the sequential sum is redone over x.
__device__ __forceinline__ float rms_scale(double S, const float* x, int n, float eps) {
    const double dn = (double)n;
    const double err = S * (4.0 * dn * 0x1p-53);
    const float lo = (float)((S - err) / dn), hi = (float)((S + err) / dn);
    float mean = lo;
    if (!(lo == hi)) {
        double q = 0.0;
        for (int i = 0; i < n; i++) q += (double)x[i] * (double)x[i];
        mean = (float)(q / dn);
    }
    return 1.0f / sqrtf(mean + eps);
}

// One Q8_K block {f32 d, i8 qs[256], i16 bsums[16]} from one whole wave, lane l
// holding elements 4l..4l+3: amax over the block (exact in any order), d =
// amax / 127, id = 127 / amax (0 when amax is 0), q = rint(x * id), bsums of
// 16 consecutive q.  yb is 4-byte aligned.
__device__ __forceinline__ void q8k_wave_store(float4 v, uint8_t* __restrict__ yb, int lane) {
    float amax = fmaxf(fmaxf(abs_no_nan(v.x), abs_no_nan(v.y)), fmaxf(abs_no_nan(v.z), abs_no_nan(v.w)));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror
    amax = fmaxf(amax, dpp_f<0x140>(amax));  // row_mirror: every lane holds its 16-lane row's max
    amax = fmaxf(fmaxf(readlane_f(amax, 0), readlane_f(amax, 16)), fmaxf(readlane_f(amax, 32), readlane_f(amax, 48)));
    const float d = amax / 127.0f;
    const float id = q8_id(amax);
    const int q0 = (int)__builtin_rintf(v.x * id), q1 = (int)__builtin_rintf(v.y * id);
    const int q2 = (int)__builtin_rintf(v.z * id), q3 = (int)__builtin_rintf(v.w * id);
    const uint32_t packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
                            ((uint32_t)(q3 & 0xFF) << 24);
    *reinterpret_cast<uint32_t*>(yb + 4 + 4 * lane) = packed;
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<0xB1>(s);
    s += dpp_i<0x4E>(s);
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(yb + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *reinterpret_cast<float*>(yb) = d;
}

}  // namespace bpdq
