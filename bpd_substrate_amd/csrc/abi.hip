// abi.hip — the exported C ABI (include/bpdq.h): argument validation, error
// recording, stream selection and the launches.  Nothing here computes on the
// CPU: every numeric result comes from a gfx950 kernel.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/bpdq.h"
#include "bpdq_launch.h"

namespace {

thread_local int g_err = BPDQ_OK;
thread_local char g_msg[256] = "";
hipStream_t g_stream = nullptr;

void set_err(int code, const char* fn, const char* what) {
    if (g_err == BPDQ_OK) g_err = code;
    std::snprintf(g_msg, sizeof g_msg, "%s: %s", fn, what);
}

bool hip_ok(hipError_t e, const char* fn) {
    if (e == hipSuccess) return true;
    set_err(BPDQ_ERR_HIP, fn, hipGetErrorString(e));
    return false;
}

// After a launch: report launch-configuration errors without synchronizing.
void check_launch(const char* fn) { hip_ok(hipGetLastError(), fn); }

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Validation shared by the entry points.  Returns false (and records why) if
// nothing should be launched; `empty` is set when there is no work.
struct Check {
    const char* fn;
    bool ok = true;
    explicit Check(const char* f) : fn(f) {}
    Check& nonneg(int v, const char* name) {
        if (ok && v < 0) fail(BPDQ_ERR_SHAPE, name, "is negative");
        return *this;
    }
    Check& multiple(int v, int m, const char* name) {
        if (ok && v % m != 0) {
            char buf[96];
            std::snprintf(buf, sizeof buf, "%s=%d is not a multiple of %d", name, v, m);
            set_err(BPDQ_ERR_SHAPE, fn, buf);
            ok = false;
        }
        return *this;
    }
    Check& ptr(const void* p, uintptr_t align, const char* name) {
        if (!ok) return *this;
        if (p == nullptr) fail(BPDQ_ERR_NULL, name, "is NULL");
        else if (!aligned(p, align)) {
            char buf[96];
            std::snprintf(buf, sizeof buf, "%s is not %d-byte aligned", name, (int)align);
            set_err(BPDQ_ERR_ALIGN, fn, buf);
            ok = false;
        }
        return *this;
    }
    void fail(int code, const char* name, const char* what) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "%s %s", name, what);
        set_err(code, fn, buf);
        ok = false;
    }
};

// Device workspaces for the quantized activations of the fp32-input entry
// points (the reference mallocs one per call, bench/bpd_cpu.c:4300,4441).
// There is one per (device, stream): calls on one stream run in order and may
// share a buffer, calls on different streams get different buffers.  A caller
// keeps the entry locked (WsLease) from its request until its launches are
// enqueued, so two host threads on one stream cannot interleave their quantize
// and GEMM launches over one buffer.
//
// A buffer is never freed while its entry lives.  When a request outgrows it, a
// new buffer (at least twice the old size, so the buffers kept add up to less
// than twice the largest) becomes current and the old one is kept on the
// entry's retired list: a HIP graph captured earlier holds the old address and
// may still be replayed, on any stream.  Only bpd_gpu_workspace_release(), which
// the caller makes once no captured graph uses the stream's buffers, frees them.
// Inside graph capture nothing is allocated: a request that does not fit fails
// with BPDQ_ERR_CAPTURE (run the call once outside capture first).
//
// Entries are never deleted, only recycled (dev = -1 marks a free entry), so a
// pointer taken from the table stays valid; the lease re-checks the entry's
// owner once it holds the entry's lock.
constexpr int kWsEntries = 64;
constexpr int kWsRetired = 32;  // growths per entry: doubling from 1 MiB passes any device's memory first
struct WsEntry {
    int dev = -1;
    hipStream_t stream = nullptr;
    std::mutex mu;
    void* p = nullptr;
    size_t bytes = 0;
    void* retired[kWsRetired] = {};
    int n_retired = 0;
};
std::mutex g_ws_table_mu;
WsEntry* g_ws_table[kWsEntries];
int g_ws_count = 0;

WsEntry* ws_find(int dev, hipStream_t s) {
    for (int i = 0; i < g_ws_count; i++)
        if (g_ws_table[i]->dev == dev && g_ws_table[i]->stream == s) return g_ws_table[i];
    return nullptr;
}

// Whether e still belongs to (dev, s); the caller holds e->mu (lock order: an
// entry's lock, then the table's).
bool ws_owned(WsEntry* e, int dev, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_ws_table_mu);
    return e->dev == dev && e->stream == s;
}

WsEntry* ws_entry(int dev, hipStream_t s, const char* fn) {
    std::lock_guard<std::mutex> lk(g_ws_table_mu);
    if (WsEntry* e = ws_find(dev, s)) return e;
    for (int i = 0; i < g_ws_count; i++)
        if (g_ws_table[i]->dev == -1) {  // a released entry: its lock may still be held by a
            WsEntry* e = g_ws_table[i];  // lease that re-checks the owner and retries
            e->dev = dev;
            e->stream = s;
            return e;
        }
    if (g_ws_count == kWsEntries) {
        set_err(BPDQ_ERR_ALLOC, fn,
                "more than 64 (device, stream) workspaces: release those of finished streams with "
                "bpd_gpu_workspace_release");
        return nullptr;
    }
    WsEntry* e = new WsEntry;  // lives until the process ends
    e->dev = dev;
    e->stream = s;
    g_ws_table[g_ws_count++] = e;
    return e;
}

}  // namespace

namespace bpdq {
WsLease workspace(size_t bytes, hipStream_t s, const char* fn) {
    WsLease L;
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), fn)) return L;
    WsEntry* e = nullptr;
    for (;;) {  // the entry may be released and recycled between lookup and lock
        e = ws_entry(dev, s, fn);
        if (!e) return L;
        L.lock = std::unique_lock<std::mutex>(e->mu);
        if (ws_owned(e, dev, s)) break;
        L.lock.unlock();
    }
    if (bytes <= e->bytes) {
        L.ptr = e->p;
        return L;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!hip_ok(hipStreamIsCapturing(s, &cs), fn)) return L;
    if (cs != hipStreamCaptureStatusNone) {
        set_err(BPDQ_ERR_CAPTURE, fn, "the workspace must grow, which cannot happen during stream capture");
        return L;
    }
    if (e->p != nullptr && e->n_retired == kWsRetired) {
        set_err(BPDQ_ERR_ALLOC, fn, "the stream's workspace grew 32 times: release it with bpd_gpu_workspace_release");
        return L;
    }
    size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);  // whole MiB
    if (want < 2 * e->bytes) want = 2 * e->bytes;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        set_err(BPDQ_ERR_ALLOC, fn, "workspace allocation failed");
        return L;
    }
    if (e->p != nullptr) e->retired[e->n_retired++] = e->p;  // kept for graphs captured with it
    e->p = p;
    e->bytes = want;
    L.ptr = e->p;
    return L;
}
}  // namespace bpdq

namespace {

// Frees every buffer of (current device, s) after the whole device is idle (a
// graph captured on s may have been replayed on another stream), and recycles
// the entry.
void workspace_release(hipStream_t s, const char* fn) {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), fn)) return;
    WsEntry* e = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_ws_table_mu);
        e = ws_find(dev, s);
    }
    if (e == nullptr) return;  // nothing was ever allocated for it
    std::unique_lock<std::mutex> lk(e->mu);  // waits for a lease that is enqueueing
    if (!ws_owned(e, dev, s)) return;  // released meanwhile
    if (!hip_ok(hipDeviceSynchronize(), fn)) return;
    for (int i = 0; i < e->n_retired; i++) hip_ok(hipFree(e->retired[i]), fn);
    if (e->p != nullptr) hip_ok(hipFree(e->p), fn);
    e->n_retired = 0;
    e->p = nullptr;
    e->bytes = 0;
    std::lock_guard<std::mutex> tl(g_ws_table_mu);
    e->dev = -1;
    e->stream = nullptr;
}

void dequant_q4k(const uint8_t* q, float* out, int nb, int order, const char* fn) {
    Check c(fn);
    c.nonneg(nb, "n_blocks");
    if (!c.ok || nb == 0) return;
    c.ptr(q, 16, "q").ptr(out, 16, "out");
    if (!c.ok) return;
    bpdq::launch_dequant_q4k(q, out, nb, order, g_stream);
    check_launch(fn);
}

void* alloc(int bytes, const char* fn) {
    if (bytes < 0) {
        set_err(BPDQ_ERR_SHAPE, fn, "bytes is negative");
        return nullptr;
    }
    if (bytes == 0) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)bytes) != hipSuccess) {
        (void)hipGetLastError();
        set_err(BPDQ_ERR_ALLOC, fn, "hipMalloc failed");
        return nullptr;
    }
    return p;
}

void copy(void* dst, const void* src, int bytes, hipMemcpyKind kind, const char* fn) {
    Check c(fn);
    c.nonneg(bytes, "bytes");
    if (!c.ok || bytes == 0) return;
    c.ptr(dst, 1, "dst").ptr(src, 1, "src");
    if (!c.ok) return;
    hip_ok(hipMemcpy(dst, src, (size_t)bytes, kind), fn);
}

void dequant_q6k(const uint8_t* q, float* out, int nb, int order, const char* fn) {
    Check c(fn);
    c.nonneg(nb, "n_blocks");
    if (!c.ok || nb == 0) return;
    c.ptr(q, 2, "q").ptr(out, 16, "out");
    if (!c.ok) return;
    bpdq::launch_dequant_q6k(q, out, nb, order, g_stream);
    check_launch(fn);
}

void q6k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, const char* fn) {
    Check c(fn);
    c.nonneg(M, "M").nonneg(K, "K").multiple(K, 256, "K");
    if (!c.ok || M == 0) return;
    c.ptr(y, 4, "y");
    if (K > 0) c.ptr(w, 2, "w").ptr(xq, 4, "xq");
    if (!c.ok) return;
    bpdq::launch_qmatmul_q6k_q8k(w, xq, y, M, K, order, g_stream);
    check_launch(fn);
}

void q4k_q8k(const uint8_t* w, const uint8_t* xq, float* y, int M, int K, int order, const char* fn) {
    Check c(fn);
    c.nonneg(M, "M").nonneg(K, "K").multiple(K, 256, "K");
    if (!c.ok || M == 0) return;
    c.ptr(y, 4, "y");
    if (K > 0) c.ptr(w, 16, "w").ptr(xq, 4, "xq");
    if (!c.ok) return;
    bpdq::launch_qmatmul_q4k_q8k(w, xq, y, M, K, order, g_stream);
    check_launch(fn);
}

// List arguments of the multi-matrix GEMVs.  Returns true when there is work.
bool check_multi(Check& c, const uint8_t* const* w_list, float* const* y_list, const int* M_list, int n, int K) {
    if (n < 0 || n > 4) c.fail(BPDQ_ERR_SHAPE, "n", "is outside 0..4");
    c.nonneg(K, "K").multiple(K, 256, "K");
    if (!c.ok || n == 0) return false;
    c.ptr(w_list, 1, "w_list").ptr(y_list, 1, "y_list").ptr(M_list, 1, "M_list");
    if (!c.ok) return false;
    int rows = 0;
    for (int i = 0; i < n && c.ok; i++) {
        c.nonneg(M_list[i], "M_list[i]");
        if (!c.ok || M_list[i] == 0) continue;
        rows += M_list[i];
        c.ptr(y_list[i], 4, "y_list[i]");
        if (K > 0) c.ptr(w_list[i], 16, "w_list[i]");
    }
    return c.ok && rows > 0;
}

// Q4_K x Q8_K(x) with the quantization of fp32 x inside the GEMV kernel.
// Beyond the fused kernel's K it quantizes into the workspace first (same bits).
void fused(const uint8_t* const* w_list, float* const* y_list, const int* M_list, int n, const float* x, int K,
           const char* fn) {
    Check c(fn);
    if (!check_multi(c, w_list, y_list, M_list, n, K)) return;
    if (K > 0) c.ptr(x, 16, "x");
    if (!c.ok) return;
    if (K == 0) {
        bpdq::launch_qmatmul_q4k_q8k_multi(w_list, y_list, M_list, n, nullptr, 0, 0, g_stream);
    } else if (K <= bpdq::fused_max_k()) {
        bpdq::launch_qmatmul_q4k_fused_multi(w_list, y_list, M_list, n, x, K, 0, g_stream);
    } else {
        bpdq::WsLease ws = bpdq::workspace((size_t)(K / 256) * 292, g_stream, fn);
        uint8_t* xq = static_cast<uint8_t*>(ws.ptr);
        if (!xq) return;
        bpdq::launch_quant_q8k(x, xq, K, g_stream);
        bpdq::launch_qmatmul_q4k_q8k_multi(w_list, y_list, M_list, n, xq, K, 0, g_stream);
    }
    check_launch(fn);
}

}  // namespace

namespace bpdq {
void abi_error(int code, const char* fn, const char* what) { set_err(code, fn, what); }
bool abi_hip_ok(hipError_t e, const char* fn) { return hip_ok(e, fn); }
hipStream_t abi_stream() { return g_stream; }
}  // namespace bpdq

extern "C" {

int bpd_gpu_last_error(void) {
    const int e = g_err;
    g_err = BPDQ_OK;
    return e;
}

const char* bpd_gpu_last_error_message(void) { return g_msg; }

void bpd_gpu_set_stream(void* s) { g_stream = static_cast<hipStream_t>(s); }

void bpd_gpu_workspace_release(void* s) { workspace_release(static_cast<hipStream_t>(s), "bpd_gpu_workspace_release"); }

// ---- Q4_K -------------------------------------------------------------------
void bpd_dequant_q4k_gpu(const uint8_t* q, float* out, int n_blocks) {
    dequant_q4k(q, out, n_blocks, 0, "bpd_dequant_q4k_gpu");
}

void bpd_dequant_q4k_gguf_gpu(const uint8_t* q, float* out, int n_blocks) {
    dequant_q4k(q, out, n_blocks, 1, "bpd_dequant_q4k_gguf_gpu");
}

void bpd_qmatmul_q4k_gpu(const uint8_t* w, const float* x, float* y, int M, int K) {
    const char* fn = "bpd_qmatmul_q4k_gpu";
    Check c(fn);
    c.nonneg(M, "M").nonneg(K, "K").multiple(K, 256, "K");
    if (!c.ok || M == 0) return;
    c.ptr(y, 4, "y");
    if (K > 0) c.ptr(w, 16, "w").ptr(x, 4, "x");
    if (!c.ok) return;
    bpdq::launch_qmatmul_q4k_chain(w, x, y, M, K, g_stream);
    check_launch(fn);
}

void bpd_quant_q8_k_gpu(const float* x, uint8_t* y, int n) {
    const char* fn = "bpd_quant_q8_k_gpu";
    Check c(fn);
    c.nonneg(n, "n").multiple(n, 256, "n");
    if (!c.ok || n == 0) return;
    c.ptr(x, 16, "x").ptr(y, 4, "y");
    if (!c.ok) return;
    bpdq::launch_quant_q8k(x, y, n, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q4k_q8k_gpu(const uint8_t* w, const uint8_t* xq, float* y, int M, int K) {
    q4k_q8k(w, xq, y, M, K, 0, "bpd_qmatmul_q4k_q8k_gpu");
}

void bpd_qmatmul_q4k_q8k_gguf_gpu(const uint8_t* w, const uint8_t* xq, float* y, int M, int K) {
    q4k_q8k(w, xq, y, M, K, 1, "bpd_qmatmul_q4k_q8k_gguf_gpu");
}

void bpd_qmatmul_q4k_q8k_multi_gpu(const uint8_t* const* w_list, float* const* y_list, const int* M_list, int n,
                                   const uint8_t* xq, int K) {
    const char* fn = "bpd_qmatmul_q4k_q8k_multi_gpu";
    Check c(fn);
    if (!check_multi(c, w_list, y_list, M_list, n, K)) return;
    if (K > 0) c.ptr(xq, 4, "xq");
    if (!c.ok) return;
    bpdq::launch_qmatmul_q4k_q8k_multi(w_list, y_list, M_list, n, xq, K, 0, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q4k_q8k_fused_multi_gpu(const uint8_t* const* w_list, float* const* y_list, const int* M_list, int n,
                                         const float* x, int K) {
    fused(w_list, y_list, M_list, n, x, K, "bpd_qmatmul_q4k_q8k_fused_multi_gpu");
}

void bpd_qmatmul_q4k_q8k_fused_gpu(const uint8_t* w, const float* x, float* y, int M, int K) {
    fused(&w, &y, &M, 1, x, K, "bpd_qmatmul_q4k_q8k_fused_gpu");
}

// ---- Q6_K --------------------------------------------------------------------
void bpd_dequant_q6k_gpu(const uint8_t* q, float* out, int n_blocks) {
    dequant_q6k(q, out, n_blocks, 0, "bpd_dequant_q6k_gpu");
}
void bpd_dequant_q6k_gguf_gpu(const uint8_t* q, float* out, int n_blocks) {
    dequant_q6k(q, out, n_blocks, 1, "bpd_dequant_q6k_gguf_gpu");
}
void bpd_qmatmul_q6k_q8k_gpu(const uint8_t* w, const uint8_t* xq, float* y, int M, int K) {
    q6k_q8k(w, xq, y, M, K, 0, "bpd_qmatmul_q6k_q8k_gpu");
}
void bpd_qmatmul_q6k_q8k_gguf_gpu(const uint8_t* w, const uint8_t* xq, float* y, int M, int K) {
    q6k_q8k(w, xq, y, M, K, 1, "bpd_qmatmul_q6k_q8k_gguf_gpu");
}

// ---- the reference Python loader's per-type fp32 (load_tensor_by_type) ---------
void bpd_dequant_gguf_py_gpu(const uint8_t* src, float* out, int64_t n_elements, int ggml_type) {
    const char* fn = "bpd_dequant_gguf_py_gpu";
    Check c(fn);
    int per = 0;
    switch (ggml_type) {
        case 0:
        case 1: per = 1; break;
        case 2: per = 32; break;
        case 10:
        case 11:
        case 12:
        case 14: per = 256; break;
        default: {
            char buf[96];
            std::snprintf(buf, sizeof buf, "ggml_type %d has no loader formula", ggml_type);
            set_err(BPDQ_ERR_SHAPE, fn, buf);
            return;
        }
    }
    if (n_elements < 0) return c.fail(BPDQ_ERR_SHAPE, "n_elements", "is negative");
    if (n_elements % per != 0) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "n_elements=%lld is not a multiple of %d", (long long)n_elements, per);
        set_err(BPDQ_ERR_SHAPE, fn, buf);
        return;
    }
    if (ggml_type == 14 && n_elements / 256 > INT_MAX) return c.fail(BPDQ_ERR_SHAPE, "n_elements", "is too large");
    if (n_elements == 0) return;
    c.ptr(src, ggml_type == 14 ? 2 : 1, "src").ptr(out, 16, "out");
    if (!c.ok) return;
    bpdq::launch_dequant_gguf_py(src, out, n_elements, ggml_type, g_stream);
    check_launch(fn);
}

// ---- Q8 padded 64-byte layout (the reference's dp4a weight layout) -----------
void bpd_q8_pad64_from_f32_gpu(const float* x, uint8_t* out, int N, int K) {
    const char* fn = "bpd_q8_pad64_from_f32_gpu";
    Check c(fn);
    c.nonneg(N, "N").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || N == 0 || K == 0) return;
    c.ptr(x, 4, "x").ptr(out, 4, "out");
    if (!c.ok) return;
    bpdq::launch_q8_pad64(x, out, N, K, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q8_pad64_gpu(const uint8_t* Wp, const uint8_t* Xq, float* out, int m_weight, int m_tokens, int K) {
    const char* fn = "bpd_qmatmul_q8_pad64_gpu";
    Check c(fn);
    c.nonneg(m_weight, "m_weight").nonneg(m_tokens, "m_tokens").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || m_weight == 0 || m_tokens == 0) return;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(Wp, 4, "W_pad64").ptr(Xq, 1, "X_q8_0");
    if (!c.ok) return;
    bpdq::launch_q8_pad64_dispatch_T(Wp, Xq, out, m_weight, m_tokens, K, g_stream);
    check_launch(fn);
}

void* qgpu_alloc(int bytes) { return alloc(bytes, "qgpu_alloc"); }
void qgpu_free(void* p) {
    if (p) hip_ok(hipFree(p), "qgpu_free");
}
void qgpu_h2d(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyHostToDevice, "qgpu_h2d"); }
void qgpu_d2h(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyDeviceToHost, "qgpu_d2h"); }
void qgpu_sync(void) { hip_ok(hipDeviceSynchronize(), "qgpu_sync"); }

// ---- sweep / head-to-head aliases ---------------------------------------------
void dequant_v1_256(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_v1_256"); }
void dequant_v1_128(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_v1_128"); }
void dequant_v1_64(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_v1_64"); }
void dequant_v1_32(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_v1_32"); }
void dequant_ilp2(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_ilp2"); }
void dequant_multi2(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_multi2"); }
void dequant_multi4(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_multi4"); }
void dequant_multi8(const uint8_t* q, float* o, int nb) { dequant_q4k(q, o, nb, 0, "dequant_multi8"); }
void* sgpu_alloc(int bytes) { return alloc(bytes, "sgpu_alloc"); }
void sgpu_free(void* p) {
    if (p) hip_ok(hipFree(p), "sgpu_free");
}
void sgpu_h2d(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyHostToDevice, "sgpu_h2d"); }
void sgpu_d2h(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyDeviceToHost, "sgpu_d2h"); }
void sgpu_sync(void) { hip_ok(hipDeviceSynchronize(), "sgpu_sync"); }

void run_llamacpp(const void* q, float* o, int nb) {
    dequant_q4k(static_cast<const uint8_t*>(q), o, nb, 1, "run_llamacpp");
}
void run_bpd(const void* q, float* o, int nb) { dequant_q4k(static_cast<const uint8_t*>(q), o, nb, 1, "run_bpd"); }
void* galloc(int bytes) { return alloc(bytes, "galloc"); }
void gfree(void* p) {
    if (p) hip_ok(hipFree(p), "gfree");
}
void gh2d(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyHostToDevice, "gh2d"); }
void gd2h(void* d, const void* s, int bytes) { copy(d, s, bytes, hipMemcpyDeviceToHost, "gd2h"); }
void gsync(void) { hip_ok(hipDeviceSynchronize(), "gsync"); }

// ---- Q8_0 ---------------------------------------------------------------------
void bpd_dequant_q8_0_gpu(const uint8_t* raw, float* out, int n_blocks) {
    const char* fn = "bpd_dequant_q8_0_gpu";
    Check c(fn);
    c.nonneg(n_blocks, "n_blocks");
    if (!c.ok || n_blocks == 0) return;
    c.ptr(raw, 1, "raw").ptr(out, 4, "out");
    if (!c.ok) return;
    bpdq::launch_dequant_q8_0(raw, out, n_blocks, g_stream);
    check_launch(fn);
}

void bpd_embed_lookup_q8_0_gpu(const uint8_t* table, const int32_t* ids, float* out, int n_tokens, int embed_dim) {
    const char* fn = "bpd_embed_lookup_q8_0_gpu";
    Check c(fn);
    c.nonneg(n_tokens, "n_tokens").nonneg(embed_dim, "embed_dim").multiple(embed_dim, 32, "embed_dim");
    if (!c.ok || n_tokens == 0 || embed_dim == 0) return;
    c.ptr(table, 1, "table").ptr(ids, 4, "token_ids").ptr(out, 4, "out");
    if (!c.ok) return;
    bpdq::launch_embed_q8_0(table, ids, out, n_tokens, embed_dim, g_stream);
    check_launch(fn);
}

void bpd_quant_q8_0_gpu(const float* x, uint8_t* y, int n_elements) {
    const char* fn = "bpd_quant_q8_0_gpu";
    Check c(fn);
    c.nonneg(n_elements, "n_elements").multiple(n_elements, 32, "n_elements");
    if (!c.ok || n_elements == 0) return;
    c.ptr(x, 4, "x").ptr(y, 1, "y");
    if (!c.ok) return;
    bpdq::launch_quant_q8_0(x, y, n_elements, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q8_0_dispatch_gpu(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens,
                                   int K) {
    const char* fn = "bpd_qmatmul_q8_0_dispatch_gpu";
    Check c(fn);
    c.nonneg(m_weight, "m_weight").nonneg(m_tokens, "m_tokens").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || m_weight == 0 || m_tokens == 0) return;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(Wq, 1, "W_q8_0").ptr(Xq, 1, "X_q8_0");
    if (!c.ok) return;
    bpdq::launch_q8_0_dispatch_T(Wq, Xq, out, m_weight, m_tokens, K, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q8_0_llamafile_gpu(const uint8_t* W, const float* X, float* out, int m_weight, int m_tokens, int K) {
    const char* fn = "bpd_qmatmul_q8_0_llamafile_gpu";
    Check c(fn);
    c.nonneg(m_weight, "m_weight").nonneg(m_tokens, "m_tokens").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || m_weight == 0 || m_tokens == 0) return;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(W, 1, "W_q8_0").ptr(X, 4, "X_f32");
    if (!c.ok) return;
    const size_t xq_bytes = (size_t)m_tokens * (size_t)(K / 32) * 34;
    bpdq::WsLease ws;
    uint8_t* xq = nullptr;
    if (xq_bytes > 0) {
        ws = bpdq::workspace(xq_bytes, g_stream, fn);
        xq = static_cast<uint8_t*>(ws.ptr);
        if (!xq) return;
        // K % 32 == 0, so the flat m_tokens*K array quantizes to the same blocks as row by row.
        bpdq::launch_quant_q8_0(X, xq, (int64_t)m_tokens * K, g_stream);
        check_launch(fn);
    }
    bpdq::launch_q8_0_dispatch_T(W, xq, out, m_weight, m_tokens, K, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q8_0_dispatch_s_gpu(const uint8_t* Wq, const uint8_t* Xq, float* out, int m_weight, int m_tokens,
                                     int K) {
    const char* fn = "bpd_qmatmul_q8_0_dispatch_s_gpu";
    Check c(fn);
    c.nonneg(m_weight, "m_weight").nonneg(m_tokens, "m_tokens").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || m_weight == 0 || m_tokens == 0) return;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(Wq, 1, "W_q8_0").ptr(Xq, 1, "X_q8_0");
    if (!c.ok) return;
    bpdq::launch_q8_0_gemm_S(Wq, Xq, out, m_weight, m_tokens, K, 0, g_stream);
    check_launch(fn);
}

void bpd_qmatmul_q8_0_llamafile_s_gpu(const uint8_t* W, const float* X, float* out, int m_weight, int m_tokens,
                                      int K) {
    const char* fn = "bpd_qmatmul_q8_0_llamafile_s_gpu";
    Check c(fn);
    c.nonneg(m_weight, "m_weight").nonneg(m_tokens, "m_tokens").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || m_weight == 0 || m_tokens == 0) return;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(W, 1, "W_q8_0").ptr(X, 4, "X_f32");
    if (!c.ok) return;
    const size_t xq_bytes = (size_t)m_tokens * (size_t)(K / 32) * 34;
    bpdq::WsLease ws;
    uint8_t* xq = nullptr;
    if (xq_bytes > 0) {
        ws = bpdq::workspace(xq_bytes, g_stream, fn);
        xq = static_cast<uint8_t*>(ws.ptr);
        if (!xq) return;
        bpdq::launch_quant_q8_0(X, xq, (int64_t)m_tokens * K, g_stream);
    }
    bpdq::launch_q8_0_gemm_S(W, xq, out, m_weight, m_tokens, K, 1, g_stream);
    check_launch(fn);
}

// ---- bpd_qmm_q4k, the qdot grid and bpd_qmatmul_q8_0_cpu's form -----------------
void bpd_qmm_q4k_gpu(const uint8_t* A, const float* B, float* C, int M, int N, int K) {
    const char* fn = "bpd_qmm_q4k_gpu";
    Check c(fn);
    c.nonneg(M, "M").nonneg(N, "N").nonneg(K, "K").multiple(K, 256, "K");
    if (!c.ok || M == 0 || N == 0) return;
    c.ptr(C, 4, "C");
    if (K > 0) c.ptr(A, 16, "A").ptr(B, 4, "B");
    if (!c.ok) return;
    bpdq::launch_qmm_q4k(A, B, C, M, N, K, g_stream);
    check_launch(fn);
}

// out[m*N + n] = one qdot of weight row n and activation row m (order P or S).
static void qdot_grid(const uint8_t* Wq, const uint8_t* Xq, float* out, int M, int N, int K, bool p_order, const char* fn) {
    if (p_order && K > bpdq::qdot_p_max_k()) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "K=%d is above the %d the staged activation row holds", K, bpdq::qdot_p_max_k());
        set_err(BPDQ_ERR_LIMIT, fn, buf);
        return;
    }
    if (p_order)
        bpdq::launch_q8_0_qdot_P(Wq, Xq, out, N, M, K, g_stream);
    else
        bpdq::launch_q8_0_gemm_S(Wq, Xq, out, N, M, K, 1, g_stream);
    check_launch(fn);
}

static bool check_qdot_args(Check& c, const void* W, const void* X, const float* out, int M, int N, int K, uintptr_t xa) {
    c.nonneg(M, "M").nonneg(N, "N").nonneg(K, "K").multiple(K, 32, "K");
    if (!c.ok || M == 0 || N == 0) return false;
    c.ptr(out, 4, "out");
    if (K > 0) c.ptr(W, 1, "W").ptr(X, xa, "X");
    return c.ok;
}

void bpd_qdot_q8_0_q8_0_grid_gpu(const uint8_t* Wq, const uint8_t* Xq, float* out, int M, int N, int K) {
    const char* fn = "bpd_qdot_q8_0_q8_0_grid_gpu";
    Check c(fn);
    if (check_qdot_args(c, Wq, Xq, out, M, N, K, 1)) qdot_grid(Wq, Xq, out, M, N, K, true, fn);
}

void bpd_qdot_q8_0_q8_0_grid_s_gpu(const uint8_t* Wq, const uint8_t* Xq, float* out, int M, int N, int K) {
    const char* fn = "bpd_qdot_q8_0_q8_0_grid_s_gpu";
    Check c(fn);
    if (check_qdot_args(c, Wq, Xq, out, M, N, K, 1)) qdot_grid(Wq, Xq, out, M, N, K, false, fn);
}

// The prefill's gate/up with SwiGLU in the epilogue (order S), for tests and
// measurement: yq = Q8_0(silu(Xq . Wg) * (Xq . Wu)), M token rows of F/32 blocks.
void bpdq_q8_0_gemm_swiglu_s_gpu(const uint8_t* Wg, const uint8_t* Wu, const uint8_t* Xq, uint8_t* yq, int M, int F,
                                 int K) {
    const char* fn = "bpdq_q8_0_gemm_swiglu_s_gpu";
    Check c(fn);
    c.nonneg(M, "M").nonneg(F, "F").nonneg(K, "K").multiple(F, 64, "F").multiple(K, 128, "K");
    if (!c.ok || M == 0 || F == 0) return;
    c.ptr(Wg, 4, "Wg").ptr(Wu, 4, "Wu").ptr(Xq, 4, "Xq").ptr(yq, 2, "yq");
    if (!c.ok) return;
    if (K == 0) {
        c.fail(BPDQ_ERR_SHAPE, "K", "must be positive");
        return;
    }
    bpdq::launch_q8_0_gemm_S_swiglu(Wg, Wu, F, Xq, M, K, 1, yq, g_stream);
    check_launch(fn);
}

// bpd_qmatmul_q8_0_cpu (bench/bpd_cpu.c:4295-4315): quantize the M rows of X, then the qdot grid.
static void qmatmul_q8_0(const uint8_t* W, const float* X, float* out, int M, int N, int K, bool p_order, const char* fn) {
    Check c(fn);
    if (!check_qdot_args(c, W, X, out, M, N, K, 4)) return;
    if (p_order && K > bpdq::qdot_p_max_k()) {
        qdot_grid(nullptr, nullptr, out, M, N, K, true, fn);  // records the limit
        return;
    }
    const size_t xq_bytes = (size_t)M * (size_t)(K / 32) * 34;
    bpdq::WsLease ws;
    uint8_t* xq = nullptr;
    if (xq_bytes > 0) {
        ws = bpdq::workspace(xq_bytes, g_stream, fn);
        xq = static_cast<uint8_t*>(ws.ptr);
        if (!xq) return;
        bpdq::launch_quant_q8_0(X, xq, (int64_t)M * K, g_stream);
    }
    qdot_grid(W, xq, out, M, N, K, p_order, fn);
}

void bpd_qmatmul_q8_0_gpu(const uint8_t* W, const float* X, float* out, int M, int N, int K) {
    qmatmul_q8_0(W, X, out, M, N, K, true, "bpd_qmatmul_q8_0_gpu");
}

void bpd_qmatmul_q8_0_s_gpu(const uint8_t* W, const float* X, float* out, int M, int N, int K) {
    qmatmul_q8_0(W, X, out, M, N, K, false, "bpd_qmatmul_q8_0_s_gpu");
}

// ---- measurement helper ---------------------------------------------------------
void bpdq_stream_read_gpu(const uint8_t* p, int n16, uint32_t* sink) {
    const char* fn = "bpdq_stream_read_gpu";
    Check c(fn);
    c.nonneg(n16, "n16");
    if (!c.ok || n16 == 0) return;
    c.ptr(p, 16, "p").ptr(sink, 4, "sink");
    if (!c.ok) return;
    bpdq::launch_stream_read(p, n16, sink, g_stream);
    check_launch(fn);
}

void bpdq_stream_write_gpu(uint8_t* p, int n16, uint32_t value) {
    const char* fn = "bpdq_stream_write_gpu";
    Check c(fn);
    c.nonneg(n16, "n16");
    if (!c.ok || n16 == 0) return;
    c.ptr(p, 16, "p");
    if (!c.ok) return;
    bpdq::launch_stream_write(p, n16, value, g_stream);
    check_launch(fn);
}

void bpdq_mfma_i8_probe_gpu(int waves, int iters, uint32_t* sink) {
    const char* fn = "bpdq_mfma_i8_probe_gpu";
    Check c(fn);
    c.nonneg(waves, "waves").nonneg(iters, "iters").multiple(waves, 4, "waves");
    if (c.ok && waves > (1 << 20)) c.fail(BPDQ_ERR_SHAPE, "waves", "is above 2^20");
    if (!c.ok || waves == 0) return;
    c.ptr(sink, 4, "sink");
    if (!c.ok) return;
    bpdq::launch_mfma_i8_probe(waves, iters, sink, g_stream);
    check_launch(fn);
}

}  // extern "C"
