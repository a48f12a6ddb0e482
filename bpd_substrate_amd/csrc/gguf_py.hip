// gguf_py.hip — the reference Python loader's per-type fp32 dequant on the GPU.
//
//   k_dequant_py<TYPE>   Q4_0, Q2_K, Q3_K, Q4_K blocks -> fp32
//   k_copy_f16_f32<F16>  F16 (numpy's astype) or F32 (a copy) -> fp32
//
// load_tensor_by_type (inference/llamatov_helpers.py:196-222) turns each GGUF
// tensor into fp32 with numpy float32 arithmetic, and its driver re-quantizes
// every matrix to the padded Q8 layout (inference/llamatov_c_inference.py:
// 136-161).  The element maps and the operation order here are the Python's:
//   F16  (:205-207) astype: exact, a NaN keeps its payload and signalling bit;
//   Q4_0 (:71-98)   {f16 d, qs[16]}: element e < 16 low nibble of qs[e], 16 + e
//                   the high one; y = d * (q - 8);
//   Q2_K (:25-39)   {scales[16], qs[64], f16 d, f16 dmin}: q = bits 2(e%4)..+1 of
//                   qs[e/4]; y = ((scales[e/16] & 15) * d) * q - (scales[e/16] >> 4) * dmin;
//   Q3_K (:42-68)   the reference's approximate form, {hmask[32], qs[64],
//                   scales[12], f16 d}: scale i = (scales[i % 8] nibble i / 8) - 8,
//                   quant = q + 4 * (bit e%8 of hmask[e/8]) - 4, y = (d * scale) * quant;
//   Q4_K (:101-158) the 6-bit scales of bench/bpd_quant.c:56-62 and the Python's
//                   own map: element e < 128 low nibble of qs[e] in sub-block e/32,
//                   128 + e high nibble in sub-block 4 + e/32;
//                   y = ((d * sc) * q) - (dmin * m).
// Each product and difference is one fp32 operation with the Python
// expression's left operand first; where it is NaN, x86's bits (numpy runs on
// x86 SSE/AVX): the first NaN operand quieted, else the default NaN.  Q6_K is
// k_dequant_q6k<0> (q6k.hip), which already follows :161-179.
//
// One thread per 4 consecutive outputs (a 16-byte store); block bytes by byte
// loads, so no source alignment is needed.  A one-time load path: HBM-bound
// and not tuned further.
// ----------------------------------------------------------------------------
#include "bpdq_launch.h"
#include "bpdq_device.h"

namespace bpdq {

// numpy's float16 -> float32: exact for finite values; Inf / NaN get exponent
// 255 and the payload shifted up, with no quiet bit added.
__device__ __forceinline__ float f16_numpy(uint32_t h) {
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31u) return __uint_as_float(s | 0x7F800000u | (m << 13));
    if (e == 0u) return __uint_as_float(__float_as_uint((float)m * 0x1p-24f) | s);  // exact: m < 2^10
    return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
}

__device__ __forceinline__ float mul_x86(float first, float second) {
    const float r = first * second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}
__device__ __forceinline__ float sub_x86(float first, float second) {
    const float r = first - second;
    return __builtin_isnan(r) ? x86_nan_of(first, second) : r;
}

__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

template <int TYPE>
struct PyBlock;
template <>
struct PyBlock<2> {
    static constexpr int kBytes = 18, kPer = 32;
};
template <>
struct PyBlock<10> {
    static constexpr int kBytes = 84, kPer = 256;
};
template <>
struct PyBlock<11> {
    static constexpr int kBytes = 110, kPer = 256;
};
template <>
struct PyBlock<12> {
    static constexpr int kBytes = 144, kPer = 256;
};

template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant_py(const uint8_t* __restrict__ q, float* __restrict__ out,
                                                    int64_t n_quads) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n_quads) return;
    constexpr int QPB = PyBlock<TYPE>::kPer / 4;  // quads per block
    const uint8_t* blk = q + (t / QPB) * PyBlock<TYPE>::kBytes;
    const int e0 = (int)(t % QPB) * 4;
    float v[4];
    if constexpr (TYPE == 2) {  // Q4_0
        const float d = f16_numpy(rd16(blk));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = e0 + i;
            const int x = e < 16 ? blk[2 + e] & 15 : blk[2 + e - 16] >> 4;
            v[i] = mul_x86(d, (float)x - 8.0f);
        }
    } else if constexpr (TYPE == 10) {  // Q2_K
        const float d = f16_numpy(rd16(blk + 80)), dm = f16_numpy(rd16(blk + 82));
        const uint32_t sb = blk[e0 >> 4], qb = blk[16 + (e0 >> 2)];
        const float sc = mul_x86((float)(sb & 15u), d), mn = mul_x86((float)(sb >> 4), dm);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = sub_x86(mul_x86(sc, (float)((qb >> (2 * i)) & 3u)), mn);
    } else if constexpr (TYPE == 11) {  // Q3_K (the reference's approximate form)
        const float d = f16_numpy(rd16(blk + 108));
        const int si = e0 >> 4;
        const uint32_t sbyte = blk[96 + (si & 7)];
        const float ds = mul_x86(d, (float)(si < 8 ? sbyte & 15u : sbyte >> 4) - 8.0f);
        const uint32_t qb = blk[32 + (e0 >> 2)], hb = blk[e0 >> 3] >> (e0 & 7);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float quant = (float)((qb >> (2 * i)) & 3u) + (float)((hb >> i) & 1u) * 4.0f - 4.0f;
            v[i] = mul_x86(ds, quant);
        }
    } else {  // Q4_K, the Python map
        const float d = f16_numpy(rd16(blk)), dmin = f16_numpy(rd16(blk + 2));
        const int hi = e0 >= 128, ii = e0 & 127, j = (hi ? 4 : 0) + (ii >> 5);
        const uint8_t* s = blk + 4;
        const int sc = j < 4 ? s[j] & 63 : (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        const int m = j < 4 ? s[j + 4] & 63 : (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        const float dsc = mul_x86(d, (float)sc), dm = mul_x86(dmin, (float)m);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t b = blk[16 + ii + i];
            v[i] = sub_x86(mul_x86(dsc, (float)(hi ? b >> 4 : b & 15u)), dm);
        }
    }
    reinterpret_cast<float4*>(out)[t] = make_float4(v[0], v[1], v[2], v[3]);
}

// F16 (numpy's astype) or F32 (bit copy) -> fp32, 4 elements per thread; the
// last thread takes the n % 4 tail element by element.
template <bool F16>
__global__ __launch_bounds__(256) void k_copy_f16_f32(const uint8_t* __restrict__ src, float* __restrict__ out,
                                                      int64_t n) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x, e0 = 4 * t;
    if (e0 >= n) return;
    const int cnt = n - e0 < 4 ? (int)(n - e0) : 4;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i < cnt) {
            const uint8_t* p = src + (e0 + i) * (F16 ? 2 : 4);
            v[i] = F16 ? f16_numpy(rd16(p)) : __uint_as_float(rd16(p) | (rd16(p + 2) << 16));
        }
    }
    if (cnt == 4) {
        reinterpret_cast<float4*>(out)[t] = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        for (int i = 0; i < cnt; i++) out[e0 + i] = v[i];
    }
}

static int64_t quads_grid(int64_t quads) { return (quads + 255) / 256; }

bool launch_dequant_gguf_py(const uint8_t* src, float* out, int64_t n_elements, int ggml_type, hipStream_t s) {
    switch (ggml_type) {
        case 0:
        case 1: {
            const int64_t q = (n_elements + 3) / 4;
            if (ggml_type == 0)
                hipLaunchKernelGGL(k_copy_f16_f32<false>, dim3(quads_grid(q)), dim3(256), 0, s, src, out, n_elements);
            else
                hipLaunchKernelGGL(k_copy_f16_f32<true>, dim3(quads_grid(q)), dim3(256), 0, s, src, out, n_elements);
            return true;
        }
        case 2:
            hipLaunchKernelGGL(k_dequant_py<2>, dim3(quads_grid(n_elements / 4)), dim3(256), 0, s, src, out,
                               n_elements / 4);
            return true;
        case 10:
            hipLaunchKernelGGL(k_dequant_py<10>, dim3(quads_grid(n_elements / 4)), dim3(256), 0, s, src, out,
                               n_elements / 4);
            return true;
        case 11:
            hipLaunchKernelGGL(k_dequant_py<11>, dim3(quads_grid(n_elements / 4)), dim3(256), 0, s, src, out,
                               n_elements / 4);
            return true;
        case 12:
            hipLaunchKernelGGL(k_dequant_py<12>, dim3(quads_grid(n_elements / 4)), dim3(256), 0, s, src, out,
                               n_elements / 4);
            return true;
        case 14:
            launch_dequant_q6k(src, out, (int)(n_elements / 256), 0, s);
            return true;
        default:
            return false;
    }
}

}  // namespace bpdq
