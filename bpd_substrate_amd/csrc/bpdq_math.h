// bpdq_math.h — device restatement of the C library's expf, so the decode
// step's softmax and SiLU round exactly as the reference's CPU code does.
//
// The reference calls expf from the platform libm (bench/bpd_cpu.c:5414 in
// bpd_gqa_attn_cpu, :5521 in bpd_swiglu_fuse_cpu).  On x86-64 glibc (2.27 and
// later) that is the table-driven method of Szabolcs Nagy, published in ARM's
// optimized-routines (math/expf.c, math/exp2f_data.c), in the variant glibc
// selects on CPUs with FMA:
//   z = N/ln2 * x;  k = round(z) via the 1.5*2^52 shift;  r = z - k   (both FMA)
//   2^(k/N) from a 32-entry table with the exponent added in integer form
//   exp(x) ~= 2^(k/N) * (C0 r^3 + C1 r^2 + C2 r + 1)                  (FMA)
// computed in binary64 and rounded once to binary32.
// tab[i] = bits(RN64(2^(i/32))) - (i << 52)/32, i.e. the correctly rounded
// binary64 value of 2^(i/32) with i/32 taken out of its exponent field; the
// polynomial coefficients are the published ones, each divided by N^j.
// A plain-C copy of the same steps agrees with glibc's expf on every one of the
// 2^32 binary32 inputs that is not a NaN (checked exhaustively by the tests).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bpdq {

static __constant__ uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab: the 32 entries of kExp2fTab, wherever the caller keeps them (a kernel
// with many exps per lane copies them to LDS: a per-lane index into constant
// memory is a vector load from the cache hierarchy for every call).
//
// Branch-free: the main steps run for every input (the table index is masked,
// so any input reads inside the table), and the special results of |x| >= 88
// replace them by selects, so a lane's exps are straight-line code that the
// compiler can interleave (branches per exp serialize each table read).
__device__ __forceinline__ float expf_libm(float x, const uint64_t* tab = kExp2fTab) {
    constexpr double kN = 32.0;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / (kN * kN * kN);
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / (kN * kN);
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab[ki & 31] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    float out = (float)y;
    // The empty asm takes the main result and x together and hands both on, so
    // the selects below depend on the main steps and the compiler cannot sink
    // those steps into a branch taken only when no special case applies.
    float xs = x;
    asm("" : "+v"(out), "+v"(xs));
    // |x| >= 88, Inf or NaN (each condition below implies it): underflow, overflow,
    // +Inf and NaN (x + x), -Inf (0), in the order that lets the later one win
    out = xs < -0x1.9fe368p6f ? 0.0f : out;
    out = xs > 0x1.62e42ep6f ? __uint_as_float(0x7f800000u) : out;
    out = abstop >= 0x7f8u ? xs + xs : out;
    out = ux == 0xff800000u ? 0.0f : out;
    return out;
}

}  // namespace bpdq
