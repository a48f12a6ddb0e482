// noalloc.hip — bpd_qmatmul_q8_0_llamafile_noalloc_gpu: the llamafile entry
// (quantize fp32 X to Q8_0 rows, then the tile-order dispatcher) for callers
// that cannot allocate device memory: code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc.
//
// The Q8_0 rows of X go to `scratch`, a fixed device array of kScratchBytes
// that every GPU the library runs on holds for the life of the process.  On the
// host the array's name is only a stand-in symbol, never a device address, so
// host code never passes it to a kernel: the first call on each device, with
// that device current, looks up that device's address with hipGetSymbolAddress
// and keeps it; every launch takes that pointer.  Nothing here calls hipMalloc,
// hipFree or any other allocating routine.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, or two host threads) race on it.  The quantizer writes every
// byte the GEMM reads, so nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/bpdq.h"
#include "bpdq_launch.h"

namespace {

constexpr size_t kScratchBytes = (size_t)8 << 20;  // 8 MiB: 512 tokens x K = 14336 fit (7.3 MiB)
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];  // device address of `scratch` per device, nullptr until looked up

// This device's address of `scratch` (looked up on first use), or nullptr with
// the error recorded.
uint8_t* scratch_ptr(const char* fn) {
    int dev = 0;
    if (!bpdq::abi_hip_ok(hipGetDevice(&dev), fn)) return nullptr;
    if (dev < 0 || dev >= kMaxDevices) {
        bpdq::abi_error(BPDQ_ERR_LIMIT, fn, "device ordinal beyond the 64 the scratch table holds");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        if (!bpdq::abi_hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), fn)) return nullptr;
        g_scratch_dev[dev] = p;
    }
    return static_cast<uint8_t*>(g_scratch_dev[dev]);
}

}  // namespace

extern "C" {

void bpd_qmatmul_q8_0_llamafile_noalloc_gpu(const uint8_t* W, const float* X, float* out, int m_weight,
                                            int m_tokens, int K) {
    const char* fn = "bpd_qmatmul_q8_0_llamafile_noalloc_gpu";
    if (m_weight < 0 || m_tokens < 0 || K < 0) {
        bpdq::abi_error(BPDQ_ERR_SHAPE, fn, "negative size");
        return;
    }
    if (K % 32 != 0) {
        bpdq::abi_error(BPDQ_ERR_SHAPE, fn, "K is not a multiple of 32");
        return;
    }
    if (m_weight == 0 || m_tokens == 0) return;
    if (out == nullptr || (K > 0 && (W == nullptr || X == nullptr))) {
        bpdq::abi_error(BPDQ_ERR_NULL, fn, "NULL pointer for a non-empty tensor");
        return;
    }
    if ((reinterpret_cast<uintptr_t>(out) & 3) != 0 || (reinterpret_cast<uintptr_t>(X) & 3) != 0) {
        bpdq::abi_error(BPDQ_ERR_ALIGN, fn, "X and out must be 4-byte aligned");
        return;
    }
    const size_t xq_bytes = (size_t)m_tokens * (size_t)(K / 32) * 34;
    if (xq_bytes > kScratchBytes) {
        char msg[160];
        std::snprintf(msg, sizeof msg, "X needs %zu bytes of Q8_0 rows, above the %zu-byte scratch array", xq_bytes,
                      kScratchBytes);
        bpdq::abi_error(BPDQ_ERR_LIMIT, fn, msg);
        return;
    }
    const hipStream_t s = bpdq::abi_stream();
    uint8_t* xq = nullptr;
    if (xq_bytes > 0) {
        xq = scratch_ptr(fn);
        if (xq == nullptr) return;
        bpdq::launch_quant_q8_0(X, xq, (int64_t)m_tokens * K, s);
    }
    bpdq::launch_q8_0_dispatch_T(W, xq, out, m_weight, m_tokens, K, s);
    bpdq::abi_hip_ok(hipGetLastError(), fn);
}

}  // extern "C"
