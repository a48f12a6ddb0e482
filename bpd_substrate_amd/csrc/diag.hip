// diag.hip — measurement helpers (no counterpart in the reference).
//
// k_stream_read: the fastest plain HBM read of n16 16-byte pieces found on this
// device for a single launch: each wave reads a contiguous run of 288 pieces
// (4,608 bytes, lane l taking pieces l, l+64, ...) with non-temporal loads, the
// load pattern of the span GEMV without its arithmetic, and stores once per wave
// only if the data XORs to a magic value.  It gives the streaming-read floor of
// a single launch of a given size, and a kernel of exactly known traffic for
// calibrating the FETCH_SIZE counter.  k_stream_write and k_mfma_i8_probe (below)
// give the write floor and the int8 MFMA rate.  Measured for 33.0 MB: 5.87 us, against
// 6.38 us for one plain 16-byte load per lane and 6.02 us for the same with
// the non-temporal hint.
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

constexpr int kReadRun = 288;                  // pieces per wave
constexpr int kReadLoads = (kReadRun + 63) / 64;

__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, int64_t n16,
                                                     uint32_t* __restrict__ sink) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int64_t run = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kReadRun;
    v4 v[kReadLoads];
    // lanes past the run or the buffer repeat its last piece (the same line: no
    // extra traffic), so that every load is unconditional
#pragma unroll
    for (int u = 0; u < kReadLoads; u++) {
        const int64_t j = min(run + min(lane + 64 * u, kReadRun - 1), n16 - 1);
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p + j));
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kReadLoads; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

void launch_stream_read(const uint8_t* p, int64_t n16, uint32_t* sink, hipStream_t s) {
    const int64_t runs = (n16 + kReadRun - 1) / kReadRun;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)((runs + 3) / 4)), dim3(256), 0, s,
                       reinterpret_cast<const uint4*>(p), n16, sink);
}

// k_stream_write: the write counterpart: each wave stores a contiguous run of
// 288 16-byte pieces (lane l taking pieces l, l+64, ...) with non-temporal
// stores, every piece once.  The single-launch HBM write floor of a given size
// (the dequant kernels write 7 bytes for every byte they read).
__global__ __launch_bounds__(256) void k_stream_write(uint4* __restrict__ p, int64_t n16, uint32_t value) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int64_t run = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kReadRun;
    const v4 v = {value, value ^ (uint32_t)lane, value, (uint32_t)run};
#pragma unroll
    for (int u = 0; u < kReadLoads; u++) {
        const int64_t j = run + lane + 64 * u;
        if (lane + 64 * u < kReadRun && j < n16) __builtin_nontemporal_store(v, reinterpret_cast<v4*>(p + j));
    }
}

void launch_stream_write(uint8_t* p, int64_t n16, uint32_t value, hipStream_t s) {
    const int64_t runs = (n16 + kReadRun - 1) / kReadRun;
    hipLaunchKernelGGL(k_stream_write, dim3((unsigned)((runs + 3) / 4)), dim3(256), 0, s, reinterpret_cast<uint4*>(p),
                       n16, value);
}

// k_mfma_i8_probe: the int8 matrix rate of the device.  Every wave runs `iters`
// rounds of 4 independent v_mfma_i32_32x32x32_i8 accumulations on register
// operands (no memory traffic), 4 * 32*32*32 * 2 = 262,144 int8 ops per round,
// and stores once only if its accumulators fold to a magic value.
__global__ __launch_bounds__(256) void k_mfma_i8_probe(int iters, uint32_t* __restrict__ sink) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    typedef int i16 __attribute__((ext_vector_type(16)));
    const int lane = threadIdx.x & 63;
    i4 a = {lane, lane * 3, lane ^ 0x55, iters};
    i4 b = {lane * 7, lane + 11, lane ^ 0x2A, 5};
    i16 c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
    }
    int f = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) f ^= c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
    if ((uint32_t)f == 0x9E3779B9u) sink[0] = (uint32_t)f;
}

// 4 waves per workgroup, `waves` waves in all (a multiple of 4).
void launch_mfma_i8_probe(int waves, int iters, uint32_t* sink, hipStream_t s) {
    hipLaunchKernelGGL(k_mfma_i8_probe, dim3((unsigned)(waves / 4)), dim3(256), 0, s, iters, sink);
}

}  // namespace bpdq
