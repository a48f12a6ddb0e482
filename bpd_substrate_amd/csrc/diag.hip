// diag.hip — measurement helpers (no counterpart in the reference).
//
// k_stream_read: the simplest full-rate HBM read of n16 16-byte chunks (one
// 16-byte load per lane, grid covering the buffer once, one store per wave that
// only happens if the data XORs to a magic value).  It gives the streaming-read
// floor of a single launch of a given size on this device, and a kernel of
// exactly known traffic for calibrating the FETCH_SIZE counter.
#include "bpdq_device.h"
#include "bpdq_launch.h"

namespace bpdq {

__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, int64_t n16,
                                                     uint32_t* __restrict__ sink) {
    const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int64_t j = i + 256 * u;
        v[u] = j < n16 ? p[j] : make_uint4(0, 0, 0, 0);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

void launch_stream_read(const uint8_t* p, int64_t n16, uint32_t* sink, hipStream_t s) {
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)((n16 + 1023) / 1024)), dim3(256), 0, s,
                       reinterpret_cast<const uint4*>(p), n16, sink);
}

}  // namespace bpdq
