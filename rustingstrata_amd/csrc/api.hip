// The C ABI (include/strata_hip.h): context, memory, argument checks, and the launch sequences of the hot-path
// Backend methods (src/backend.rs:98-443, CUDA implementation src/cuda/mod.rs:748-1242).
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.h"
#include "moe.h"
#include "gemm.h"
#include "decoder.h"
#include "../../include/strata_hip.h"

using namespace strata;

namespace strata {

static thread_local std::string g_err;

int set_error(const std::string& msg) {
    g_err = msg;
    return -1;
}
int hip_error(hipError_t e, const char* what) {
    return set_error(std::string("HIP error ") + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ") in " + what);
}
const char* type_name(int ty) {
    switch (ty) {
    case Q8_0: return "Q8_0";
    case Q2_K: return "Q2_K";
    case Q3_K: return "Q3_K";
    case Q4_K: return "Q4_K";
    case Q5_K: return "Q5_K";
    case Q6_K: return "Q6_K";
    case IQ2_XXS: return "IQ2_XXS";
    case IQ3_S: return "IQ3_S";
    case IQ4_XS: return "IQ4_XS";
    }
    return "unknown";
}

// Device scratch that grows on demand. Growing waits for the stream first: queued kernels may still read it. A
// recorded graph keeps the addresses it was recorded with, so a buffer replaced while any graph of the context
// exists is retired, not freed, until the last graph is destroyed (or the context closes); while the stream is
// recording, scratch cannot grow at all (the wait would end the recording).
struct Scratch {
    void* p = nullptr;
    size_t n = 0;
    std::vector<void*> retired;
    hipError_t need(size_t bytes, hipStream_t s, bool recording, bool graphs_alive) {
        if (bytes <= n) return hipSuccess;
        if (recording) return hipErrorStreamCaptureUnsupported;
        if (p) {
            hipError_t e = hipStreamSynchronize(s);
            if (e != hipSuccess) return e;
            if (graphs_alive) retired.push_back(p);
            else hipFree(p);
            p = nullptr;
            n = 0;
        }
        size_t want = std::max(bytes, (size_t)1 << 20);
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) return e;
        n = want;
        return hipSuccess;
    }
    void free_retired() {
        for (void* q : retired) hipFree(q);
        retired.clear();
    }
    void release() {
        free_retired();
        if (p) hipFree(p);
        p = nullptr;
        n = 0;
    }
};

// Scratch of strata_gemvn_noalloc: the quantized x of up to 4 inputs of up to 16384 values (int8 values, then one
// f32 scale per 32), in a file-scope device array so that the call allocates nothing. Each GPU holds its own copy
// until the process ends; host code reaches it only through the address hipGetSymbolAddress returns for the device.
constexpr size_t NOALLOC_SCRATCH_BYTES = 4 * (16384 + 16384 / 8);
static __device__ __align__(256) int8_t scratch[NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch_ptr;  // device -> address of `scratch` on it

// The device address of `scratch` on `device` (current), looked up once per device.
hipError_t noalloc_scratch(int device, void** out) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    auto it = g_scratch_ptr.find(device);
    if (it != g_scratch_ptr.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = ptr;
    *out = ptr;
    return hipSuccess;
}

}  // namespace strata

struct strata_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int numerics = STRATA_NUM_Q8K;
    std::mutex mu;
    std::map<uint64_t, size_t> allocs;  // start -> bytes
    Scratch xq;                          // quantized x of GEMV calls that pass none
    Scratch gx;                          // quantized x of the GEMM (kept for SAME_X)
    uint64_t gx_key[4] = {0, 0, 0, 0};   // x, x_stride, n_x, cols of gx's contents (all 0: none)
    Scratch misc;
    Scratch am;                          // argmax partials
    void* noalloc = nullptr;             // this device's address of the file-scope `scratch`
    bool recording = false;              // between strata_graph_begin and strata_graph_end
    int graphs = 0;                      // executable graphs made by this context and not yet destroyed
    hipError_t need(Scratch& s, size_t bytes) { return s.need(bytes, stream, recording, graphs > 0); }
};

namespace {

int check_ctx(strata_ctx* c) {
    if (!c) return set_error("null strata context");
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_error(e, "hipSetDevice");
    return 0;
}

// The allocation of this context holding [a, a + n).
bool in_alloc(strata_ctx* c, uint64_t a, size_t n) {
    std::lock_guard<std::mutex> g(c->mu);
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return false;
    --it;
    return a >= it->first && a + n <= it->first + it->second && a + n >= a;
}

int check_type(int ty) {
    if (!supported(ty))
        return set_error("unsupported quant type (ggml type id " + std::to_string(ty) +
                         "); this backend decodes Q8_0 Q2_K Q3_K Q4_K Q5_K Q6_K IQ2_XXS IQ3_S IQ4_XS");
    return 0;
}

// Gpu::gemv_cols (src/cuda/mod.rs:567-571), with this backend's requirement of whole 256-value super-blocks for the
// K and IQ types (the reference's `_p` kernels cover partial ones; no hot-path shape has them).
int check_gemv_cols(int ty, uint64_t cols, bool wide) {
    uint64_t b = ty == Q8_0 ? 32 : 256;
    if (cols == 0 || cols % b)
        return set_error(std::string(type_name(ty)) + " tensor with " + std::to_string(cols) +
                         " columns: GEMV needs a multiple of " + std::to_string(b));
    if (row_bytes(ty, cols) > gemv_max_row_bytes())
        return set_error(std::string(type_name(ty)) + " tensor with " + std::to_string(cols) +
                         " columns: a row exceeds the GEMV tile (" + std::to_string(gemv_max_row_bytes()) + " bytes)");
    if (!wide && cols > GEMV1_MAX_COLS)
        return set_error("GEMV with " + std::to_string(cols) + " columns: at most " + std::to_string(GEMV1_MAX_COLS) +
                         " on this path (gemv / gemvn / gemvq take wider rows)");
    return 0;
}

// Weight address alignment the decoders assume (super-block start alignment mod 16).
int check_align(int ty, uint64_t addr, const char* what) {
    uint64_t a = ty == Q4_K || ty == Q5_K ? 16 : ty == IQ4_XS ? 8 : ty == Q2_K ? 4 : 2;
    if (addr % a)
        return set_error(std::string(what) + ": " + type_name(ty) + " weights at a " + std::to_string(addr % a) +
                         "-misaligned address (need " + std::to_string(a) + "-byte alignment)");
    return 0;
}

// Quantize x (nt rows, x_stride apart) into the context's GEMV scratch; returns the scratch address.
int quant_into_scratch(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t n, uint64_t nt, uint64_t* out) {
    STRATA_HIP(c->need(c->xq, xq_bytes(n, nt)));
    STRATA_HIP(launch_quant_xq((const float*)x, x_stride, (int)n, (int)nt, (int8_t*)c->xq.p, c->numerics, c->stream));
    *out = (uint64_t)c->xq.p;
    return 0;
}

int check_tensor(const strata_tensor* w, const char* what) {
    if (!w) return set_error(std::string(what) + ": null tensor");
    if (check_type(w->ty)) return -1;
    if (!w->ptr && w->rows) return set_error(std::string(what) + ": null weight address");
    return 0;
}

}  // namespace

extern "C" {

const char* strata_last_error(void) { return g_err.c_str(); }

int strata_open(int device, strata_ctx** out) {
    if (!out) return set_error("strata_open: null out");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return set_error("strata_open: GPU " + std::to_string(device) + " of " + std::to_string(n));
    STRATA_HIP(hipSetDevice(device));
    strata_ctx* c = new strata_ctx();
    c->device = device;
    e = noalloc_scratch(device, &c->noalloc);
    if (e != hipSuccess) { delete c; return hip_error(e, "hipGetSymbolAddress(scratch)"); }
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) { delete c; return hip_error(e, "hipStreamCreate"); }
    *out = c;
    return 0;
}

void strata_close(strata_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    for (auto& kv : c->allocs) hipFree((void*)kv.first);
    c->xq.release();
    c->gx.release();
    c->misc.release();
    c->am.release();
    hipStreamDestroy(c->stream);
    delete c;
}

int strata_device_name(strata_ctx* c, char* buf, size_t len) {
    if (check_ctx(c)) return -1;
    hipDeviceProp_t p;
    STRATA_HIP(hipGetDeviceProperties(&p, c->device));
    if (buf && len) {
        std::snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    }
    return 0;
}

int strata_set_numerics(strata_ctx* c, int mode) {
    if (!c) return set_error("null strata context");
    if (mode != STRATA_NUM_Q8K && mode != STRATA_NUM_Q8_32) return set_error("strata_set_numerics: mode " + std::to_string(mode));
    c->numerics = mode;
    c->gx_key[0] = c->gx_key[1] = c->gx_key[2] = c->gx_key[3] = 0;
    return 0;
}
int strata_get_numerics(strata_ctx* c) { return c ? c->numerics : -1; }

int strata_alloc(strata_ctx* c, size_t bytes, uint64_t* addr) {
    if (check_ctx(c)) return -1;
    if (!addr) return set_error("strata_alloc: null out");
    size_t n = std::max(bytes, (size_t)1);
    void* p = nullptr;
    // 256 bytes of slack past the end: kernels read weight rows in 16-byte-aligned covers, which may reach up to
    // 15 bytes past a row's last block.
    STRATA_HIP(hipMalloc(&p, ((n + 255) & ~(size_t)255) + 256));
    hipError_t e = hipMemsetAsync(p, 0, n, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) { hipFree(p); return hip_error(e, "zeroing a new buffer"); }
    {
        std::lock_guard<std::mutex> g(c->mu);
        c->allocs[(uint64_t)p] = n;
    }
    *addr = (uint64_t)p;
    return 0;
}

int strata_free(strata_ctx* c, uint64_t addr) {
    if (check_ctx(c)) return -1;
    {
        std::lock_guard<std::mutex> g(c->mu);
        auto it = c->allocs.find(addr);
        if (it == c->allocs.end()) return set_error("strata_free: not an allocation of this context");
        c->allocs.erase(it);
    }
    STRATA_HIP(hipStreamSynchronize(c->stream));
    STRATA_HIP(hipFree((void*)addr));
    return 0;
}

int strata_htod(strata_ctx* c, const void* src, uint64_t dst, size_t bytes) {
    if (check_ctx(c)) return -1;
    if (!bytes) return 0;
    if (!in_alloc(c, dst, bytes)) return set_error("htod: " + std::to_string(bytes) + " bytes outside the destination buffer");
    STRATA_HIP(hipMemcpyAsync((void*)dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    STRATA_HIP(hipStreamSynchronize(c->stream));
    return 0;
}

int strata_dtoh(strata_ctx* c, uint64_t src, void* dst, size_t bytes) {
    if (check_ctx(c)) return -1;
    if (!bytes) return 0;
    if (!in_alloc(c, src, bytes)) return set_error("dtoh: " + std::to_string(bytes) + " bytes outside the source buffer");
    STRATA_HIP(hipMemcpyAsync(dst, (const void*)src, bytes, hipMemcpyDeviceToHost, c->stream));
    STRATA_HIP(hipStreamSynchronize(c->stream));
    return 0;
}

int strata_dtod(strata_ctx* c, uint64_t src, uint64_t dst, size_t bytes) {
    if (check_ctx(c)) return -1;
    if (!bytes) return 0;
    if (!in_alloc(c, src, bytes) || !in_alloc(c, dst, bytes)) return set_error("dtod: range outside its buffer");
    STRATA_HIP(hipMemcpyAsync((void*)dst, (const void*)src, bytes, hipMemcpyDeviceToDevice, c->stream));
    return 0;
}

int strata_memset(strata_ctx* c, uint64_t dst, size_t bytes) {
    if (check_ctx(c)) return -1;
    if (!bytes) return 0;
    if (!in_alloc(c, dst, bytes)) return set_error("memset: range outside its buffer");
    STRATA_HIP(hipMemsetAsync((void*)dst, 0, bytes, c->stream));
    return 0;
}

int strata_mem_info(strata_ctx* c, size_t* free_bytes, size_t* total_bytes) {
    if (check_ctx(c)) return -1;
    size_t f = 0, t = 0;
    STRATA_HIP(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return 0;
}

int strata_sync(strata_ctx* c) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(hipStreamSynchronize(c->stream));
    return 0;
}

void* strata_stream(strata_ctx* c) { return c ? (void*)c->stream : nullptr; }

int strata_graph_begin(strata_ctx* c) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    // A SAME_X hit inside the recording must not lean on a quantization queued before it: the graph would replay
    // against whatever the GEMM-X scratch holds at launch time.
    c->gx_key[0] = c->gx_key[1] = c->gx_key[2] = c->gx_key[3] = 0;
    c->recording = true;
    return 0;
}

int strata_graph_end(strata_ctx* c, void** graph) {
    if (check_ctx(c)) return -1;
    if (!graph) return set_error("strata_graph_end: null out");
    hipGraph_t g = nullptr;
    c->recording = false;
    STRATA_HIP(hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_error(e, "hipGraphInstantiate");
    c->graphs++;
    *graph = (void*)ex;
    return 0;
}

int strata_graph_launch(strata_ctx* c, void* graph) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(hipGraphLaunch((hipGraphExec_t)graph, c->stream));
    return 0;
}

int strata_graph_destroy(strata_ctx* c, void* graph) {
    if (check_ctx(c)) return -1;
    // a replay still queued must finish before its executable graph goes (and before the caller frees its buffers)
    STRATA_HIP(hipStreamSynchronize(c->stream));
    STRATA_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
    if (c->graphs > 0 && --c->graphs == 0) {
        // No graph holds a retired scratch address any more.
        STRATA_HIP(hipStreamSynchronize(c->stream));
        c->xq.free_retired();
        c->gx.free_retired();
        c->misc.free_retired();
        c->am.free_retired();
    }
    return 0;
}

int strata_dequant(strata_ctx* c, const strata_tensor* w, uint64_t rows, uint64_t out) {
    if (check_ctx(c) || check_tensor(w, "dequant")) return -1;
    if (rows > w->rows) return set_error("dequant: " + std::to_string(rows) + " rows of a " + std::to_string(w->rows) + "-row tensor");
    uint64_t b = w->ty == Q8_0 ? 32 : 256;
    if (w->cols % b) return set_error(std::string(type_name(w->ty)) + " tensor with " + std::to_string(w->cols) + " columns: dequant needs a multiple of " + std::to_string(b));
    STRATA_HIP(launch_dequant(w->ty, (const uint8_t*)w->ptr, rows, w->cols, (float*)out, c->stream));
    return 0;
}

int strata_quant_xq(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t n, uint64_t nt, uint64_t out) {
    if (check_ctx(c)) return -1;
    if (n % 32) return set_error("quant_xq: " + std::to_string(n) + " values (a multiple of 32)");
    if (n > (1u << 30) || nt > (1u << 30) || nt * ((n + 255) / 256) > (1ull << 34)) return set_error("quant_xq: too large");
    STRATA_HIP(launch_quant_xq((const float*)x, x_stride, (int)n, (int)nt, (int8_t*)out, c->numerics, c->stream));
    return 0;
}

int strata_combine_rms_norm_q(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t ye, uint64_t wh, uint64_t k,
                              uint64_t w, uint64_t out, uint64_t out_stride, uint64_t n, uint64_t rows, float eps,
                              uint64_t xq, uint64_t res) {
    if (check_ctx(c)) return -1;
    if (!x || !w || !out || !ye || !wh) return set_error("combine_rms_norm_q: null x, w, out, ye or wh");
    if (xq && n % 32) return set_error("rms_norm_q: " + std::to_string(n) + " values (a multiple of 32 to quantize)");
    if (k == 0 || k > 4096 || n > (1u << 30) || rows > 65535) return set_error("combine_rms_norm_q: " + std::to_string(rows) + " rows of " + std::to_string(k) + " slots");
    if (x_stride != n) return set_error("combine_rms_norm_q: x rows must be n floats apart (moe_combine's layout)");
    const hipError_t e = launch_rms_norm_q((float*)x, x_stride, (const float*)w, (float*)out, out_stride, (int)n, (int)rows,
                                           eps, (int8_t*)xq, (const float*)res, c->numerics, c->stream, (const float*)ye,
                                           (const float*)wh, (int)k);
    if (e != hipErrorNotSupported) {
        STRATA_HIP(e);
        return 0;
    }
    // rows the one-round-trip form does not take: x += res, the combine, then the norm
    if (res && strata_add(c, x, res, n * rows)) return -1;
    if (strata_moe_combine(c, x, ye, wh, k, 0, 0, n, rows)) return -1;
    return strata_rms_norm_q(c, x, x_stride, w, out, out_stride, n, rows, eps, xq, 0);
}

int strata_combine_rms_norm_gemv(strata_ctx* c, uint64_t x, uint64_t res, uint64_t ye, uint64_t wh, uint64_t k,
                                 uint64_t nw, float eps, const strata_tensor* w, uint64_t x_out, uint64_t y) {
    if (check_ctx(c) || check_tensor(w, "combine_rms_norm_gemv")) return -1;
    if (!x || !nw || !y || (k && (!ye || !wh))) return set_error("combine_rms_norm_gemv: null x, nw, y, ye or wh");
    const uint64_t n = w->cols;
    if (k > 8 || n > 2048 || n % 8 || c->numerics != STRATA_NUM_Q8K ||
        ((x | res | ye | nw | x_out) % 16))
        return set_error("combine_rms_norm_gemv: one row of at most 2048 values (a multiple of 8, 16-byte aligned), "
                         "at most 8 slots, Q8_K numerics (" + std::to_string(n) + " values, " +
                         std::to_string(k) + " slots)");
    // block 0 writes x_out while the other blocks still read x, res and ye: x_out may overlap none of them
    if (x_out) {
        auto overlaps = [&](uint64_t p, uint64_t bytes) { return p && x_out < p + bytes && p < x_out + 4 * n; };
        if (overlaps(x, 4 * n) || overlaps(res, 4 * n) || overlaps(ye, 4 * n * k))
            return set_error("combine_rms_norm_gemv: x_out overlaps x, res or ye");
    }
    if (check_gemv_cols(w->ty, w->cols, false) || check_align(w->ty, w->ptr, "combine_rms_norm_gemv")) return -1;
    if (w->rows == 0 || w->rows > (1u << 30)) return set_error("combine_rms_norm_gemv: " + std::to_string(w->rows) + " rows");
    GemvLaunch g;
    g.xf = (const float*)x; g.x_stride = n;
    g.ty = w->ty; g.w = (const uint8_t*)w->ptr; g.rows = (int)w->rows; g.cols = (int)n;
    g.nt = 1; g.n_xrows = 1; g.y = (float*)y; g.numerics = c->numerics;
    g.nw = (const float*)nw; g.nres = (const float*)res; g.nye = (const float*)ye; g.nwh = (const float*)wh;
    g.nxw = (float*)x_out; g.neps = eps; g.nck = (int)k;
    const hipError_t e = launch_gemv(g, c->stream);
    if (e == hipErrorNotSupported) return set_error(std::string("combine_rms_norm_gemv: ") + type_name(w->ty) + " not supported");
    STRATA_HIP(e);
    return 0;
}

int strata_rms_norm_q_gemv_f32(strata_ctx* c, uint64_t x, uint64_t res, uint64_t nw, uint64_t h, uint64_t xq,
                               uint64_t n, float eps, const strata_tensor* w, uint64_t y) {
    if (check_ctx(c)) return -1;
    if (!w || !w->ptr) return set_error("rms_norm_q_gemv_f32: null matrix");
    if (!x || !res || !nw || !h || !y) return set_error("rms_norm_q_gemv_f32: null x, res, nw, h or y");
    if (w->ty != 0 || w->cols != n) return set_error("rms_norm_q_gemv_f32: an F32 matrix of " + std::to_string(n) + " columns");
    if (w->rows == 0 || w->rows >= (1ull << 31)) return set_error("rms_norm_q_gemv_f32: " + std::to_string(w->rows) + " rows");
    if (xq && n % 32) return set_error("rms_norm_q: " + std::to_string(n) + " values (a multiple of 32 to quantize)");
    const hipError_t e = launch_rms_norm_gemv_f32((const float*)x, (const float*)res, (const float*)nw, (float*)h,
                                                  (int8_t*)xq, (int)n, eps, c->numerics, (const float*)w->ptr,
                                                  (int)w->rows, (float*)y, c->stream);
    if (e == hipErrorNotSupported)
        return set_error("rms_norm_q_gemv_f32: rows of at most 2048 values, a multiple of 8, 16-byte aligned");
    STRATA_HIP(e);
    return 0;
}

int strata_rms_norm_q(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t out_stride,
                      uint64_t n, uint64_t rows, float eps, uint64_t xq, uint64_t res) {
    if (check_ctx(c)) return -1;
    if (!x || !w || !out) return set_error("rms_norm: null x, w or out");
    if (xq && n % 32) return set_error("rms_norm_q: " + std::to_string(n) + " values (a multiple of 32 to quantize)");
    if (n > (1u << 30) || rows >= (1ull << 31)) return set_error("rms_norm: too large");
    STRATA_HIP(launch_rms_norm_q((float*)x, x_stride, (const float*)w, (float*)out, out_stride, (int)n, (int)rows, eps,
                                 (int8_t*)xq, (const float*)res, c->numerics, c->stream));
    return 0;
}

int strata_rms_norm(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t out_stride, uint64_t n,
                    uint64_t rows, float eps) {
    return strata_rms_norm_q(c, x, x_stride, w, out, out_stride, n, rows, eps, 0, 0);
}

// gemv / gemm_dense of an F32 matrix (the router's ffn_gate_inp): float dots, no activation quantization.
static int gemv_f32(strata_ctx* c, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t y, uint64_t y_stride,
                    uint64_t nt, int act) {
    if (nt < 1) return set_error("gemvn: " + std::to_string(nt) + " inputs");
    if (w->cols == 0 || w->cols % 4) return set_error("F32 tensor with " + std::to_string(w->cols) + " columns: GEMV needs a multiple of 4");
    if (w->rows == 0) return 0;
    if (w->rows > (1u << 30) || w->cols > (1u << 30)) return set_error("gemv: too large");
    if (x % 16 || (nt > 1 && x_stride % 4)) return set_error("F32 gemv: x rows must be 16-byte aligned");
    STRATA_HIP(launch_gemv_f32((const float*)w->ptr, (int)w->rows, (int)w->cols, (const float*)x, x_stride, (float*)y,
                               y_stride, (int)nt, act, c->stream));
    return 0;
}

int strata_gemvq(strata_ctx* c, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t xq, uint64_t y,
                 uint64_t y_stride, uint64_t nt) {
    if (w && w->ty == STRATA_F32 && !check_ctx(c)) {
        if (nt > 4) return set_error("gemvn: " + std::to_string(nt) + " inputs (1 to 4)");
        return gemv_f32(c, w, x, x_stride, y, y_stride, nt, 0);
    }
    if (check_ctx(c) || check_tensor(w, "gemv")) return -1;
    if (nt < 1 || nt > 4) return set_error("gemvn: " + std::to_string(nt) + " inputs (1 to 4)");
    if (check_gemv_cols(w->ty, w->cols, true) || check_align(w->ty, w->ptr, "gemv")) return -1;
    if (w->rows == 0) return 0;
    if (w->rows > (1u << 30)) return set_error("gemv: too many rows");
    // One input of up to GEMV1_MAX_COLS values: the kernel quantizes x itself; several, or a wider row: quantize once
    // for all blocks.
    if (!xq && (nt > 1 || w->cols > GEMV1_MAX_COLS) && quant_into_scratch(c, x, x_stride, w->cols, nt, &xq)) return -1;
    GemvLaunch g;
    g.xf = (const float*)x; g.x_stride = x_stride;
    g.ty = w->ty; g.w = (const uint8_t*)w->ptr; g.rows = (int)w->rows; g.cols = (int)w->cols;
    g.nt = (int)nt; g.xq = (const int8_t*)xq; g.n_xrows = (int)nt; g.y = (float*)y; g.y_stride = (int)y_stride;
    g.numerics = c->numerics;
    STRATA_HIP(launch_gemv(g, c->stream));
    return 0;
}

int strata_gemv(strata_ctx* c, const strata_tensor* w, uint64_t x, uint64_t y) {
    return strata_gemvq(c, w, x, 0, 0, y, 0, 1);
}

int strata_gemvn(strata_ctx* c, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t y, uint64_t y_stride,
                 uint64_t nt) {
    return strata_gemvq(c, w, x, x_stride, 0, y, y_stride, nt);
}

int strata_gemvn_noalloc(strata_ctx* c, const strata_tensor* w, uint64_t x, uint64_t x_stride, uint64_t y,
                        uint64_t y_stride, uint64_t nt) {
    if (check_ctx(c) || check_tensor(w, "gemvn_noalloc")) return -1;
    if (nt < 1 || nt > 4) return set_error("gemvn: " + std::to_string(nt) + " inputs (1 to 4)");
    if (check_gemv_cols(w->ty, w->cols, false) || check_align(w->ty, w->ptr, "gemvn_noalloc")) return -1;
    if (nt > 1 && xq_bytes(w->cols, nt) > NOALLOC_SCRATCH_BYTES)
        return set_error("gemvn_noalloc: " + std::to_string(nt) + " inputs of " + std::to_string(w->cols) +
                         " values need " + std::to_string(xq_bytes(w->cols, nt)) + " bytes of scratch (at most " +
                         std::to_string(NOALLOC_SCRATCH_BYTES) + ")");
    if (w->rows == 0) return 0;
    if (w->rows > (1u << 30)) return set_error("gemv: too many rows");
    uint64_t xq = 0;
    if (nt > 1) {
        // Every byte the GEMV reads is written here first, so the array needs no clearing between calls.
        STRATA_HIP(launch_quant_xq((const float*)x, x_stride, (int)w->cols, (int)nt, (int8_t*)c->noalloc, c->numerics,
                                   c->stream));
        xq = (uint64_t)c->noalloc;
    }
    GemvLaunch g;
    g.xf = (const float*)x; g.x_stride = x_stride;
    g.ty = w->ty; g.w = (const uint8_t*)w->ptr; g.rows = (int)w->rows; g.cols = (int)w->cols;
    g.nt = (int)nt; g.xq = (const int8_t*)xq; g.n_xrows = (int)nt; g.y = (float*)y; g.y_stride = (int)y_stride;
    g.numerics = c->numerics;
    STRATA_HIP(launch_gemv(g, c->stream));
    return 0;
}

int strata_gemvq2(strata_ctx* c, const strata_tensor* a, const strata_tensor* b, uint64_t x, uint64_t x_stride,
                  uint64_t xq, uint64_t ya, uint64_t yb, uint64_t nt) {
    if (check_ctx(c) || check_tensor(a, "gemvq2") || check_tensor(b, "gemvq2")) return -1;
    // Different shapes or types: two launches (src/cuda/mod.rs:937-940).
    if (a->ty != b->ty || a->cols != b->cols) {
        if (strata_gemvq(c, a, x, x_stride, xq, ya, a->rows, nt)) return -1;
        return strata_gemvq(c, b, x, x_stride, xq, yb, b->rows, nt);
    }
    if (nt < 1 || nt > 4) return set_error("gemvn: " + std::to_string(nt) + " inputs (1 to 4)");
    if (a->rows > (1u << 30) || b->rows > (1u << 30)) return set_error("gemvq2: too many rows");
    if (check_gemv_cols(a->ty, a->cols, false) || check_align(a->ty, a->ptr, "gemvq2") || check_align(b->ty, b->ptr, "gemvq2")) return -1;
    if (!xq && nt > 1 && quant_into_scratch(c, x, x_stride, a->cols, nt, &xq)) return -1;
    GemvLaunch g;
    g.xf = (const float*)x; g.x_stride = x_stride;
    g.ty = a->ty; g.w = (const uint8_t*)a->ptr; g.rows = (int)a->rows; g.cols = (int)a->cols;
    g.nt = (int)nt; g.xq = (const int8_t*)xq; g.n_xrows = (int)nt; g.y = (float*)ya; g.y_stride = (int)a->rows;
    g.numerics = c->numerics;
    g.pair = true; g.w2 = (int64_t)(b->ptr - a->ptr); g.y2 = (int64_t)(yb - ya); g.rows2 = (int)b->rows;
    // The second matrix's outputs are token-strided by its own row count; one stride serves both only when equal.
    if (nt > 1 && a->rows != b->rows) {
        if (strata_gemvq(c, a, x, x_stride, xq, ya, a->rows, nt)) return -1;
        return strata_gemvq(c, b, x, x_stride, xq, yb, b->rows, nt);
    }
    STRATA_HIP(launch_gemv(g, c->stream));
    return 0;
}

// moe_gemv with x = silu(x) * xu per row when xu is not 0 (quantized in the kernel; xq must be 0 then).
static int moe_gemv_impl(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride, uint64_t ids,
                         uint64_t k, uint64_t x, uint64_t x_stride, uint64_t xg, uint64_t y, int has_pair, int64_t w2,
                         int64_t y2, uint64_t xq, uint64_t xu) {
    if (check_ctx(c) || check_type(ty)) return -1;
    if (check_gemv_cols(ty, cols, false) || check_align(ty, w, "moe_gemv")) return -1;
    if (check_align(ty, stride, "moe_gemv stride") || (has_pair && check_align(ty, (uint64_t)w2, "moe_gemv pair offset"))) return -1;
    if (xg < 1 || k % xg) return set_error("moe_gemv: " + std::to_string(k) + " slots in groups of " + std::to_string(xg));
    if (k == 0 || rows == 0) return 0;
    if (k > 65535) return set_error("moe_gemv: too many slots");
    GemvLaunch g;
    g.xf = (const float*)x; g.xu = (const float*)xu; g.x_stride = x_stride;
    g.ty = ty; g.w = (const uint8_t*)w; g.rows = (int)rows; g.cols = (int)cols; g.nt = 1;
    g.xq = (const int8_t*)xq; g.n_xrows = (int)(k / xg); g.y = (float*)y; g.y_stride = 0;
    g.numerics = c->numerics;
    g.ids = (const int*)ids; g.k = (int)k; g.xg = (int)xg; g.stride = (int64_t)stride;
    g.pair = has_pair != 0; g.w2 = w2; g.y2 = y2; g.rows2 = (int)rows;
    STRATA_HIP(launch_gemv(g, c->stream));
    return 0;
}

int strata_moe_gemv(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride, uint64_t ids,
                    uint64_t k, uint64_t x, uint64_t x_stride, uint64_t xg, uint64_t y, int has_pair, int64_t w2,
                    int64_t y2, uint64_t xq) {
    return moe_gemv_impl(c, ty, rows, cols, w, stride, ids, k, x, x_stride, xg, y, has_pair, w2, y2, xq, 0);
}

int strata_moe_route_gemv(strata_ctx* c, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t table,
                          uint64_t ids, uint64_t wts, uint64_t slots, uint64_t wh, int sigmoid, int ty, uint64_t rows,
                          uint64_t cols, uint64_t w, uint64_t stride, uint64_t x, uint64_t y, int has_pair, int64_t w2,
                          int64_t y2, uint64_t xq) {
    if (check_ctx(c) || check_type(ty)) return -1;
    if (n > 512 || k > 32 || k > n || k == 0) return set_error("moe_route_gemv: " + std::to_string(n) + " experts, top " + std::to_string(k));
    if (!table || !slots || !wh || !ids || !wts) return set_error("moe_route_gemv: null table, ids, wts, slots or wh");
    if (!rows) return strata_moe_route(c, p, n, k, extra_scale, table, ids, wts, slots, wh, 1, sigmoid);
    if (check_gemv_cols(ty, cols, false) || check_align(ty, w, "moe_route_gemv")) return -1;
    if (check_align(ty, stride, "moe_route_gemv stride") || (has_pair && check_align(ty, (uint64_t)w2, "moe_route_gemv pair offset"))) return -1;
    if (n <= 128) {
        GemvLaunch g;
        g.xf = (const float*)x; g.x_stride = cols;
        g.ty = ty; g.w = (const uint8_t*)w; g.rows = (int)rows; g.cols = (int)cols; g.nt = 1;
        g.xq = (const int8_t*)xq; g.n_xrows = 1; g.y = (float*)y; g.y_stride = 0;
        g.numerics = c->numerics;
        g.ids = (const int*)slots; g.k = (int)k; g.xg = (int)k; g.stride = (int64_t)stride;
        g.pair = has_pair != 0; g.w2 = w2; g.y2 = y2; g.rows2 = (int)rows;
        g.rp = (const float*)p; g.rn = (int)n; g.rscale = extra_scale; g.rtable = (const int*)table;
        g.rids = (int*)ids; g.rwts = (float*)wts; g.rwh = (float*)wh; g.rsig = sigmoid;
        const hipError_t e = launch_gemv(g, c->stream);
        if (e != hipErrorNotSupported) {
            STRATA_HIP(e);
            return 0;
        }
    }
    if (strata_moe_route(c, p, n, k, extra_scale, table, ids, wts, slots, wh, 1, sigmoid)) return -1;
    return strata_moe_gemv(c, ty, rows, cols, w, stride, slots, k, x, cols, k, y, has_pair, w2, y2, xq);
}

int strata_router_topk(strata_ctx* c, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t ids,
                       uint64_t wts, uint64_t t, int sigmoid) {
    if (check_ctx(c)) return -1;
    if (n > 512 || k > 32 || k > n || k == 0) return set_error("router_topk: " + std::to_string(n) + " experts, top " + std::to_string(k));
    if (!t) return 0;
    STRATA_HIP(launch_route((const float*)p, (int)n, (int)k, extra_scale, nullptr, (int*)ids, (float*)wts, nullptr,
                            nullptr, (int)t, sigmoid, c->stream));
    return 0;
}

int strata_moe_route(strata_ctx* c, uint64_t p, uint64_t n, uint64_t k, float extra_scale, uint64_t table, uint64_t ids,
                     uint64_t wts, uint64_t slots, uint64_t wh, uint64_t t, int sigmoid) {
    if (check_ctx(c)) return -1;
    if (n > 512 || k > 32 || k > n || k == 0) return set_error("moe_route: " + std::to_string(n) + " experts, top " + std::to_string(k));
    if (!table || !slots || !wh) return set_error("moe_route: null table, slots or wh");
    if (!t) return 0;
    STRATA_HIP(launch_route((const float*)p, (int)n, (int)k, extra_scale, (const int*)table, (int*)ids, (float*)wts,
                            (int*)slots, (float*)wh, (int)t, sigmoid, c->stream));
    return 0;
}

int strata_swiglu_q(strata_ctx* c, uint64_t g, uint64_t u, uint64_t n, uint64_t rows, uint64_t xq, uint64_t* ret) {
    if (check_ctx(c)) return -1;
    if (n % 32) return set_error("swiglu_q: " + std::to_string(n) + " values (a multiple of 32)");
    if (!xq) return set_error("swiglu_q: null xq");
    if (rows > (1u << 30) || n > (1u << 30) || rows * ((n + 255) / 256) > (1ull << 34))
        return set_error("swiglu_q: too large");
    STRATA_HIP(launch_swiglu_q((const float*)g, (const float*)u, (int)n, (int)rows, (int8_t*)xq, c->numerics, c->stream));
    if (ret) *ret = xq;
    return 0;
}

int strata_moe_combine(strata_ctx* c, uint64_t x, uint64_t ye, uint64_t w, uint64_t k, uint64_t sh, uint64_t sg,
                       uint64_t n, uint64_t t) {
    if (check_ctx(c)) return -1;
    if (!n || !t) return 0;
    if (t > 65535 || n > (1u << 30)) return set_error("moe_combine: too large (at most 65535 tokens a call)");
    STRATA_HIP(launch_combine((float*)x, (const float*)ye, (const float*)w, (int)k, (const float*)sh, (const float*)sg,
                              (int)n, (int)t, c->stream));
    return 0;
}

// The down GEMV and the combine as one launch where the fused layout takes the shape (1: done, 0: not taken, -1:
// error); x rows from xq.
static int down_combine_fused(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                              uint64_t slots, uint64_t k, uint64_t xq, uint64_t x, uint64_t wh, uint64_t sh, uint64_t sg,
                              uint64_t t) {
    if (check_ctx(c) || check_type(ty)) return -1;
    if (check_gemv_cols(ty, cols, false) || check_align(ty, w, "moe_down_combine") || check_align(ty, stride, "moe_down_combine stride")) return -1;
    if (!t || !rows || !k) return 1;
    if (rows > (1u << 30) || k > 256 || t > 65535 || !slots || !wh || !x) return 0;
    DownCombineLaunch d;
    d.ty = ty; d.numerics = c->numerics; d.w = (const uint8_t*)w; d.stride = (int64_t)stride;
    d.rows = (int)rows; d.cols = (int)cols; d.k = (int)k; d.t = (int)t;
    d.slots = (const int*)slots; d.wh = (const float*)wh;
    d.xq = (const int8_t*)xq;
    d.x = (float*)x; d.sh = (const float*)sh; d.sg = (const float*)sg;
    const hipError_t e = launch_down_combine(d, c->stream);
    if (e == hipErrorNotSupported) return 0;
    STRATA_HIP(e);
    return 1;
}

int strata_moe_down_combine(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                            uint64_t slots, uint64_t k, uint64_t h, uint64_t ye, uint64_t xq, uint64_t x, uint64_t wh,
                            uint64_t sh, uint64_t sg, uint64_t t) {
    if (xq) {
        const int r = down_combine_fused(c, ty, rows, cols, w, stride, slots, k, xq, x, wh, sh, sg, t);
        if (r) return r < 0 ? -1 : 0;
    }
    if (strata_moe_gemv(c, ty, rows, cols, w, stride, slots, t * k, h, cols, 1, ye, 0, 0, 0, xq)) return -1;
    return strata_moe_combine(c, x, ye, wh, k, sh, sg, rows, t);
}

int strata_moe_down_swiglu_combine(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t w, uint64_t stride,
                                   uint64_t slots, uint64_t k, uint64_t g, uint64_t u, uint64_t ye, uint64_t x,
                                   uint64_t wh, uint64_t sh, uint64_t sg, uint64_t t) {
    if (check_ctx(c)) return -1;
    if (!g || !u) return set_error("moe_down_swiglu_combine: null g or u");
    if (!x) return moe_gemv_impl(c, ty, rows, cols, w, stride, slots, t * k, g, cols, 1, ye, 0, 0, 0, 0, u);
    // (the one-launch layout would quantize every slot's SwiGLU in every block: slower than two launches)
    if (moe_gemv_impl(c, ty, rows, cols, w, stride, slots, t * k, g, cols, 1, ye, 0, 0, 0, 0, u)) return -1;
    return strata_moe_combine(c, x, ye, wh, k, sh, sg, rows, t);
}

int strata_moe_combine_seq(strata_ctx* c, uint64_t x, uint64_t ye, uint64_t wts, uint64_t inv, uint64_t k, uint64_t sh,
                           uint64_t sg, uint64_t n, uint64_t t) {
    if (check_ctx(c)) return -1;
    if (!n || !t) return 0;
    if (t > 65535 || n > (1u << 30)) return set_error("moe_combine_seq: too large (at most 65535 tokens a call)");
    STRATA_HIP(launch_combine_seq((float*)x, (const float*)ye, (const float*)wts, (const int*)inv, (int)k,
                                  (const float*)sh, (const float*)sg, (int)n, (int)t, c->stream));
    return 0;
}

int strata_moe_sort(strata_ctx* c, uint64_t ids, uint64_t t, uint64_t k, uint64_t n_expert, uint64_t off,
                    uint64_t xrow, uint64_t inv, uint64_t n_mats, const uint64_t* bases, const uint64_t* strides,
                    uint64_t tiles, uint64_t max_tiles, uint64_t n_tiles_dev, uint64_t err_dev, uint64_t chunk) {
    if (check_ctx(c)) return -1;
    if (chunk == 0) chunk = 128;
    if (chunk > 256 || chunk % 16) return set_error("moe_sort: chunk " + std::to_string(chunk) + " (a multiple of 16, at most 256)");
    if (n_expert == 0 || n_expert > 512) return set_error("moe_sort: " + std::to_string(n_expert) + " experts (1 to 512)");
    if (n_mats > 3 || (n_mats && (!bases || !strides))) return set_error("moe_sort: at most 3 matrices, with bases and strides");
    if (t * k > (1u << 30)) return set_error("moe_sort: too many pairs");
    if (max_tiles < (t * k) / chunk + n_expert)
        return set_error("moe_sort: max_tiles " + std::to_string(max_tiles) + " < pairs / chunk + experts");
    SortLaunch s;
    s.ids = (const int*)ids; s.t = (int)t; s.k = (int)k; s.n_expert = (int)n_expert;
    s.off = (int*)off; s.xrow = (int*)xrow; s.inv = (int*)inv;
    s.n_mats = (int)n_mats;
    for (uint64_t m = 0; m < n_mats; m++) { s.bases[m] = bases[m]; s.strides[m] = strides[m]; }
    s.tiles = (uint64_t*)tiles; s.max_tiles = (int)max_tiles; s.n_tiles = (int*)n_tiles_dev; s.err = (int*)err_dev;
    s.chunk = (int)chunk;
    STRATA_HIP(c->need(c->misc, sort_scratch_bytes((int)n_expert, (int)(t * k))));
    s.scratch = (int*)c->misc.p;
    STRATA_HIP(launch_sort(s, c->stream));
    return 0;
}

// GEMM X quantization, cached for SAME_X (Gpu::q8_x, src/cuda/mod.rs:626-636).
static int gemm_x(strata_ctx* c, uint64_t cols, uint64_t n_x, uint64_t x, uint64_t x_stride, int same, uint64_t* out) {
    uint64_t key[4] = {x, x_stride, n_x, cols};
    bool hit = same && std::equal(key, key + 4, c->gx_key);
    if (!hit) {
        c->gx_key[0] = c->gx_key[1] = c->gx_key[2] = c->gx_key[3] = 0;
        STRATA_HIP(c->need(c->gx, gemm_x_bytes(cols, n_x)));
        STRATA_HIP(launch_gemm_quant_x((const float*)x, x_stride, (int)cols, (int)n_x, (uint8_t*)c->gx.p, c->numerics, c->stream));
        std::copy(key, key + 4, c->gx_key);
    }
    *out = (uint64_t)c->gx.p;
    return 0;
}

static int gemm_common(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t tiles, uint64_t n_tiles,
                       const int* n_tiles_dev, uint64_t x, uint64_t x_stride, uint64_t n_x, uint64_t xrow, uint64_t y,
                       uint64_t y_stride, int act, const uint8_t* dense_w, uint64_t dense_n, bool pair = false,
                       int64_t w2 = 0) {
    if (check_ctx(c) || check_type(ty)) return -1;
    if (cols == 0 || cols % 256)
        return set_error(std::string(type_name(ty)) + " matrix with " + std::to_string(cols) + " columns: GEMM needs a multiple of 256");
    int op = act & ~(STRATA_SAME_X | STRATA_X_Q | STRATA_SMALL_TILES);
    if (op < 0 || op > 2) return set_error("gemm: act " + std::to_string(act));
    if ((act & STRATA_X_Q) && x_stride != cols) return set_error("gemm: a quantized X (STRATA_X_Q) has rows of cols values");
    if (dense_w && check_align(ty, (uint64_t)dense_w, "gemm_dense")) return -1;
    if (n_tiles == 0 || rows == 0) return 0;
    if (rows > (1u << 24) || row_bytes(ty, cols) >= (1u << 24) || n_tiles > 65535 * 64) return set_error("gemm: too large");
    if (ty == Q8_0 && n_tiles > 65535) return set_error("gemm: Q8_0 with more than 65535 tiles");
    // the kernel addresses X and a weight matrix with 32-bit byte offsets
    if (n_x * cols >= (1ull << 32) || rows * row_bytes(ty, cols) >= (1ull << 32)) return set_error("gemm: X or W of 4 GiB or more");
    uint64_t xq = x;  // STRATA_X_Q: X quantized by the caller
    if (!(act & STRATA_X_Q) && gemm_x(c, cols, n_x, x, x_stride, act & STRATA_SAME_X, &xq)) return -1;
    GemmLaunch g;
    g.ty = ty; g.rows = (int)rows; g.cols = (int)cols;
    g.tiles = (const uint64_t*)tiles; g.n_tiles = (int)n_tiles; g.n_tiles_dev = n_tiles_dev;
    g.dense_w = dense_w; g.dense_n = (int)dense_n;
    g.xq = (const uint8_t*)xq; g.n_x = (int)n_x; g.xrow = (const int*)xrow;
    g.y = (float*)y; g.y_stride = (int64_t)y_stride; g.act = op;
    g.pair = pair; g.w2 = w2;
    g.small = (act & STRATA_SMALL_TILES) != 0;
    STRATA_HIP(launch_gemm(g, c->stream));
    return 0;
}

int strata_gemm(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t tiles, uint64_t n_tiles, uint64_t x,
                uint64_t x_stride, uint64_t n_x, uint64_t xrow, uint64_t y, uint64_t y_stride, int act) {
    if (!tiles && n_tiles) return set_error("gemm: null tile list");
    return gemm_common(c, ty, rows, cols, tiles, n_tiles, nullptr, x, x_stride, n_x, xrow, y, y_stride, act, nullptr, 0);
}

int strata_gemm_grouped(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t tiles, uint64_t max_tiles,
                        uint64_t n_tiles_dev, uint64_t x, uint64_t x_stride, uint64_t n_x, uint64_t xrow, uint64_t y,
                        uint64_t y_stride, int act) {
    if (!tiles || !n_tiles_dev) return set_error("gemm_grouped: null tile list or count");
    return gemm_common(c, ty, rows, cols, tiles, max_tiles, (const int*)n_tiles_dev, x, x_stride, n_x, xrow, y, y_stride,
                       act, nullptr, 0);
}

int strata_gemm_grouped_gate_up(strata_ctx* c, int ty, uint64_t rows, uint64_t cols, uint64_t tiles,
                                uint64_t max_tiles, uint64_t n_tiles_dev, uint64_t x, uint64_t x_stride, uint64_t n_x,
                                uint64_t xrow, uint64_t y, uint64_t y_stride, int64_t up_offset, int flags) {
    if (check_ctx(c) || check_type(ty)) return -1;
    if (!tiles || !n_tiles_dev) return set_error("gemm_grouped_gate_up: null tile list or count");
    if (ty == Q8_0) return set_error("gemm_grouped_gate_up: Q8_0 has no fused gate/up kernel (use two gemm_grouped calls)");
    if (rows % 64) return set_error("gemm_grouped_gate_up: " + std::to_string(rows) + " rows (a multiple of 64)");
    if (y % 16 || y_stride % 4) return set_error("gemm_grouped_gate_up: y rows must be 16-byte aligned");
    if (check_align(ty, (uint64_t)up_offset, "gemm_grouped_gate_up up offset")) return -1;
    if (flags & ~(STRATA_SAME_X | STRATA_X_Q | STRATA_SMALL_TILES))
        return set_error("gemm_grouped_gate_up: flags " + std::to_string(flags));
    return gemm_common(c, ty, rows, cols, tiles, max_tiles, (const int*)n_tiles_dev, x, x_stride, n_x, xrow, y, y_stride,
                       flags, nullptr, 0, true, up_offset);
}

int strata_gemm_dense(strata_ctx* c, const strata_tensor* w, uint64_t n, uint64_t x, uint64_t x_stride, uint64_t y,
                      uint64_t y_stride, int act) {
    if (w && w->ty == STRATA_F32) {
        if (check_ctx(c)) return -1;
        const int op = act & ~STRATA_SAME_X;
        if (op < 0 || op > 2) return set_error("gemm: act " + std::to_string(act));
        if (w->cols == 0 || w->cols % 4 || x % 16 || x_stride % 4)
            return set_error("F32 gemm_dense: columns a multiple of 4 and x rows 16-byte aligned");
        if (n == 0 || w->rows == 0) return 0;
        if (n > (1u << 30) || w->rows > (1u << 30)) return set_error("gemm: too large");
        STRATA_HIP(launch_gemm_f32((const float*)w->ptr, (int)w->rows, (int)w->cols, (const float*)x, x_stride, (float*)y,
                                   y_stride, (int)n, op, c->stream));
        return 0;
    }
    if (check_tensor(w, "gemm_dense")) return -1;
    const uint64_t bp = gemm_block_positions();
    uint64_t nt = (n + bp - 1) / bp;
    return gemm_common(c, w->ty, w->rows, w->cols, 0, nt, nullptr, x, x_stride, n, 0, y, y_stride, act,
                       (const uint8_t*)w->ptr, n);
}

uint64_t strata_gemm_block_positions(void) { return gemm_block_positions(); }

// ---- the decoder stack ----

uint64_t strata_kv_words(uint64_t n) { return n; }

int strata_argmax_rows(strata_ctx* c, uint64_t x, uint64_t n, uint64_t rows, uint64_t out) {
    if (check_ctx(c)) return -1;
    if (!rows) return 0;
    if (n == 0 || n >= (1u << 31) || rows > 65535) return set_error("argmax_rows: " + std::to_string(rows) + " rows of " + std::to_string(n));
    STRATA_HIP(c->need(c->am, argmax_part_bytes((int)rows)));
    STRATA_HIP(launch_argmax_rows((const float*)x, (int)n, (int)rows, (uint64_t*)c->am.p, (int*)out, c->stream));
    return 0;
}

static int check_rope(uint64_t n, uint64_t n_rot) {
    if (n > 512 || n_rot > n || n_rot % 2 || n % 32 || n == 0)
        return set_error("rms_norm_rope: head of " + std::to_string(n) + ", n_rot " + std::to_string(n_rot));
    return 0;
}

int strata_rope_pairs(strata_ctx* c, uint64_t x, uint64_t stride, uint64_t heads, uint64_t per, uint64_t n_rot,
                      uint64_t step, float base, uint64_t lo, uint64_t hi) {
    if (check_ctx(c)) return -1;
    if (!per || heads % per || n_rot % 2 || n_rot > stride || hi > n_rot / 2 || lo > hi)
        return set_error("rope: " + std::to_string(heads) + " heads, " + std::to_string(per) + " per token, n_rot " +
                         std::to_string(n_rot) + ", pairs " + std::to_string(lo) + ".." + std::to_string(hi));
    if (heads >= (1u << 31)) return set_error("rope: too many heads");
    STRATA_HIP(launch_rope_pairs((float*)x, stride, (int)heads, (int)per, (int)n_rot, (const int*)step, base, (int)lo,
                                 (int)hi, c->stream));
    return 0;
}

int strata_rope_neox(strata_ctx* c, uint64_t x, uint64_t stride, uint64_t heads, uint64_t per, uint64_t n_rot,
                     uint64_t step, float base) {
    return strata_rope_pairs(c, x, stride, heads, per, n_rot, step, base, 0, n_rot / 2);
}

int strata_rms_norm_rope_qk_t(strata_ctx* c, uint64_t q, uint64_t q_tstride, uint64_t q_stride, uint64_t qw, uint64_t qo,
                              uint64_t qrows, uint64_t qper, uint64_t k, uint64_t k_tstride, uint64_t kw, uint64_t ko,
                              uint64_t krows, uint64_t kper, uint64_t n, float eps, uint64_t n_rot, uint64_t step,
                              float base, uint64_t v, uint64_t v_tstride, uint64_t kc, uint64_t vc) {
    if (check_ctx(c) || check_rope(n, n_rot)) return -1;
    if ((qrows && (!qper || qrows % qper)) || (krows && (!kper || krows % kper)))
        return set_error("rms_norm_rope: rows must be whole tokens of heads");
    if (kc && (!v || !vc)) return set_error("rms_norm_rope_kv: null v or value cache");
    if (qrows + krows >= (1u << 31)) return set_error("rms_norm_rope: too many rows");
    if ((qrows && q_tstride < qper * q_stride) || (krows && k_tstride < kper * n) || (kc && v_tstride < kper * n))
        return set_error("rms_norm_rope: a token stride shorter than its heads");
    NormRope a;
    a.x = (const float*)k; a.x_stride = n; a.x_tstride = k_tstride; a.w = (const float*)kw; a.out = (float*)ko;
    a.n = (int)n; a.rows = (int)krows; a.per = (int)(kper ? kper : 1);
    a.v = (const float*)v; a.v_tstride = v_tstride; a.kc = (uint16_t*)kc; a.vc = (uint16_t*)vc;
    a.qrows = (int)qrows; a.qx = (const float*)q; a.q_stride = q_stride; a.q_tstride = q_tstride; a.qw = (const float*)qw;
    a.qo = (float*)qo; a.qper = (int)(qper ? qper : 1);
    a.eps = eps; a.base = base; a.n_rot = (int)n_rot; a.step = (const int*)step;
    STRATA_HIP(launch_norm_rope(a, c->stream));
    return 0;
}

int strata_rms_norm_rope_qk(strata_ctx* c, uint64_t q, uint64_t q_stride, uint64_t qw, uint64_t qo, uint64_t qrows,
                            uint64_t qper, uint64_t k, uint64_t kw, uint64_t ko, uint64_t krows, uint64_t kper, uint64_t n,
                            float eps, uint64_t n_rot, uint64_t step, float base, uint64_t v, uint64_t kc, uint64_t vc) {
    if (check_ctx(c) || check_rope(n, n_rot)) return -1;
    if ((qrows && (!qper || qrows % qper)) || (krows && (!kper || krows % kper)))
        return set_error("rms_norm_rope: rows must be whole tokens of heads");
    if (kc && (!v || !vc)) return set_error("rms_norm_rope_kv: null v or value cache");
    if (qrows + krows >= (1u << 31)) return set_error("rms_norm_rope: too many rows");
    NormRope a;
    a.x = (const float*)k; a.x_stride = n; a.w = (const float*)kw; a.out = (float*)ko;
    a.n = (int)n; a.rows = (int)krows; a.per = (int)(kper ? kper : 1);
    a.v = (const float*)v; a.kc = (uint16_t*)kc; a.vc = (uint16_t*)vc;
    a.qrows = (int)qrows; a.qx = (const float*)q; a.q_stride = q_stride; a.qw = (const float*)qw; a.qo = (float*)qo;
    a.qper = (int)(qper ? qper : 1);
    a.eps = eps; a.base = base; a.n_rot = (int)n_rot; a.step = (const int*)step;
    STRATA_HIP(launch_norm_rope(a, c->stream));
    return 0;
}

int strata_rms_norm_rope_kv(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t n,
                            uint64_t rows, float eps, uint64_t per, uint64_t n_rot, uint64_t step, float base,
                            uint64_t v, uint64_t kc, uint64_t vc) {
    if (check_ctx(c) || check_rope(n, n_rot)) return -1;
    if (!per || rows % per) return set_error("rms_norm_rope: rows must be whole tokens of heads");
    if (kc && (!v || !vc)) return set_error("rms_norm_rope_kv: null v or value cache");
    if (rows >= (1u << 31)) return set_error("rms_norm_rope: too many rows");
    NormRope a;
    a.x = (const float*)x; a.x_stride = x_stride; a.w = (const float*)w; a.out = (float*)out;
    a.n = (int)n; a.rows = (int)rows; a.per = (int)per;
    a.v = (const float*)v; a.kc = (uint16_t*)kc; a.vc = (uint16_t*)vc;
    a.eps = eps; a.base = base; a.n_rot = (int)n_rot; a.step = (const int*)step;
    STRATA_HIP(launch_norm_rope(a, c->stream));
    return 0;
}

int strata_rms_norm_rope(strata_ctx* c, uint64_t x, uint64_t x_stride, uint64_t w, uint64_t out, uint64_t n,
                         uint64_t rows, float eps, uint64_t per, uint64_t n_rot, uint64_t step, float base) {
    return strata_rms_norm_rope_kv(c, x, x_stride, w, out, n, rows, eps, per, n_rot, step, base, 0, 0, 0);
}

int strata_kv_store(strata_ctx* c, uint64_t k, uint64_t v, uint64_t kc, uint64_t vc, uint64_t n, uint64_t t,
                    uint64_t step, uint64_t hd) {
    if (check_ctx(c)) return -1;
    (void)hd;  // f16 cache: the head size does not change the layout
    if (n * t >= (1ull << 40)) return set_error("kv_store: too large");
    STRATA_HIP(launch_kv_store((const float*)k, (const float*)v, (uint16_t*)kc, (uint16_t*)vc, (int)n, (int)t,
                               (const int*)step, c->stream));
    return 0;
}

static int check_attn(uint64_t nh, uint64_t nkv, uint64_t hd, const char* what) {
    if (hd != 64 && hd != 128) return set_error(std::string(what) + ": head_dim " + std::to_string(hd) + " unsupported (64 or 128)");
    if (!nkv || !nh || nh % nkv) return set_error(std::string(what) + ": " + std::to_string(nh) + " query heads over " + std::to_string(nkv) + " KV heads");
    const uint64_t g = nh / nkv;
    if (g != 1 && g != 2 && g != 4 && g != 8) return set_error(std::string(what) + ": GQA group of " + std::to_string(g) + " (1, 2, 4 or 8)");
    return 0;
}

int strata_rms_norm_rope_attn_decode(strata_ctx* c, uint64_t q, uint64_t q_stride, uint64_t qw, uint64_t k,
                                     uint64_t kw, uint64_t v, float eps, uint64_t n_rot, float base, uint64_t kc,
                                     uint64_t vc, uint64_t qg, uint64_t out, uint64_t part, uint64_t step, uint64_t nh,
                                     uint64_t nkv, uint64_t hd, float scale, uint64_t sink, uint64_t win,
                                     uint64_t xq) {
    if (check_ctx(c) || check_attn(nh, nkv, hd, "attention decode") || check_rope(hd, n_rot)) return -1;
    if (!q || !qw || !k || !kw || !v || !kc || !vc || !out || !step) return set_error("rms_norm_rope_attn_decode: null argument");
    if (!part) return set_error("attention decode: null part buffer");
    if (win >= (1u << 31)) return set_error("attention decode: too large");
    NormRope a;
    a.x = (const float*)k; a.x_stride = hd; a.w = (const float*)kw; a.n = (int)hd; a.rows = (int)nkv; a.per = (int)nkv;
    a.v = (const float*)v; a.kc = (uint16_t*)kc; a.vc = (uint16_t*)vc;
    a.qrows = (int)nh; a.qx = (const float*)q; a.q_stride = q_stride; a.qw = (const float*)qw; a.qper = (int)nh;
    a.eps = eps; a.base = base; a.n_rot = (int)n_rot; a.step = (const int*)step;
    const hipError_t e = launch_attn_decode(nullptr, (const uint16_t*)kc, (const uint16_t*)vc, (const float*)qg,
                                            (float*)out, (float*)part, (const int*)step, (int)nh, (int)nkv, (int)hd,
                                            scale, 1, (const float*)sink, (int)win, c->stream, &a, (int8_t*)xq,
                                            c->numerics);
    if (e == hipErrorNotSupported)
        return set_error("rms_norm_rope_attn_decode: q, k and v 16-byte aligned with row strides of a multiple of 4, "
                         "and nh hd a multiple of 256 with xq");
    STRATA_HIP(e);
    return 0;
}

uint64_t strata_attn_part_floats(uint64_t nh, uint64_t hd) { return nh * ATT_SPLITS * (hd + 2); }

int strata_attn_decode_gq(strata_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t part,
                          uint64_t step, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, int gq_min, uint64_t nt,
                          uint64_t sink, uint64_t win) {
    if (check_ctx(c) || check_attn(nh, nkv, hd, "attention decode")) return -1;
    (void)gq_min;  // every launch shares K / V loads across the GQA group
    if (!nt) return 0;
    if (!part) return set_error("attention decode: null part buffer");
    if (nt > 65535 || win >= (1u << 31)) return set_error("attention decode: too large");
    STRATA_HIP(launch_attn_decode((const float*)q, (const uint16_t*)kc, (const uint16_t*)vc, (const float*)qg,
                                  (float*)out, (float*)part, (const int*)step, (int)nh, (int)nkv, (int)hd, scale, (int)nt,
                                  (const float*)sink, (int)win, c->stream));
    return 0;
}

int strata_attn_decode(strata_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t part,
                       uint64_t step, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, uint64_t nt) {
    return strata_attn_decode_gq(c, q, kc, vc, qg, out, part, step, nh, nkv, hd, scale, 0, nt, 0, 0);
}

int strata_attn_prefill_m(strata_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t step,
                          uint64_t t, uint64_t nh, uint64_t nkv, uint64_t hd, float scale, uint64_t qm, uint64_t mw,
                          uint64_t sink, uint64_t win) {
    if (check_ctx(c) || check_attn(nh, nkv, hd, "attention prefill")) return -1;
    if (qm || mw) return set_error("attention prefill: QSA block masks are not supported by this backend");
    if (!t) return 0;
    if (t >= (1u << 24) || win >= (1u << 31)) return set_error("attention prefill: too large");
    if (q % 16 || out % 16 || (qg && qg % 16)) return set_error("attention prefill: q, out and qg must be 16-byte aligned");
    STRATA_HIP(launch_attn_prefill((const float*)q, (const uint16_t*)kc, (const uint16_t*)vc, (const float*)qg,
                                   (float*)out, (const int*)step, (int)t, (int)nh, (int)nkv, (int)hd, scale,
                                   (const float*)sink, (int)win, c->stream));
    return 0;
}

int strata_attn_prefill(strata_ctx* c, uint64_t q, uint64_t kc, uint64_t vc, uint64_t qg, uint64_t out, uint64_t step,
                        uint64_t t, uint64_t nh, uint64_t nkv, uint64_t hd, float scale) {
    return strata_attn_prefill_m(c, q, kc, vc, qg, out, step, t, nh, nkv, hd, scale, 0, 0, 0, 0);
}

int strata_add(strata_ctx* c, uint64_t x, uint64_t y, uint64_t n) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(launch_add((float*)x, (const float*)y, n, c->stream));
    return 0;
}

int strata_swiglu(strata_ctx* c, uint64_t g, uint64_t u, uint64_t n) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(launch_swiglu((float*)g, (const float*)u, n, c->stream));
    return 0;
}

int strata_get_rows(strata_ctx* c, const strata_tensor* w, uint64_t ids, uint64_t n, uint64_t out) {
    if (check_ctx(c) || check_tensor(w, "get_rows")) return -1;
    uint64_t b = w->ty == Q8_0 ? 32 : 256;
    if (w->cols % b || w->cols == 0) return set_error(std::string(type_name(w->ty)) + " tensor with " + std::to_string(w->cols) + " columns: get_rows needs a multiple of " + std::to_string(b));
    if (!n) return 0;
    if (!w->rows) return set_error("get_rows: empty tensor");
    if (n * (w->cols / 32) >= (1ull << 40) || n >= (1u << 31)) return set_error("get_rows: too large");
    STRATA_HIP(launch_get_rows(w->ty, (const uint8_t*)w->ptr, w->rows, w->cols, (const int*)ids, (int)n, (float*)out,
                               c->stream));
    return 0;
}

int strata_fill_blocks(strata_ctx* c, const strata_tensor* w, uint64_t seed, float lo, float hi) {
    if (check_ctx(c) || check_tensor(w, "fill_blocks")) return -1;
    if (w->cols % block_elems(w->ty)) return set_error("fill_blocks: columns not whole blocks");
    const uint64_t nb = w->rows * (w->cols / block_elems(w->ty));
    if (w->ptr % 4) return set_error("fill_blocks: the tensor must be 4-byte aligned");
    STRATA_HIP(launch_fill_blocks(w->ty, (uint8_t*)w->ptr, nb, seed, lo, hi, c->stream));
    return 0;
}

int strata_int8_gemm(strata_ctx* c, int ty) {
    (void)c;
    return supported(ty) ? 1 : 0;
}

int strata_prequant_gemm_x(strata_ctx* c, const strata_tensor* w, uint64_t n, uint64_t x, uint64_t x_stride) {
    if (check_ctx(c) || check_tensor(w, "prequant_gemm_x")) return -1;
    if (w->cols % 256) return set_error("prequant_gemm_x: " + std::to_string(w->cols) + " columns (a multiple of 256)");
    uint64_t xq;
    return gemm_x(c, w->cols, n, x, x_stride, 1, &xq);
}

uint64_t strata_row_bytes(int ty, uint64_t cols) {
    if (!supported(ty) || cols % block_elems(ty)) return 0;
    return row_bytes(ty, cols);
}

int strata_event_create(strata_ctx* c, void** ev) {
    if (check_ctx(c)) return -1;
    hipEvent_t e;
    STRATA_HIP(hipEventCreate(&e));
    *ev = (void*)e;
    return 0;
}
int strata_event_record(strata_ctx* c, void* ev) {
    if (check_ctx(c)) return -1;
    STRATA_HIP(hipEventRecord((hipEvent_t)ev, c->stream));
    return 0;
}
int strata_event_elapsed(void* start, void* end, float* ms) {
    STRATA_HIP(hipEventSynchronize((hipEvent_t)end));
    STRATA_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return 0;
}
int strata_copy_kernel(strata_ctx* c, uint64_t src, uint64_t dst, uint64_t bytes) {
    if (check_ctx(c)) return -1;
    if (bytes % 16) return set_error("copy_kernel: bytes must be a multiple of 16");
    STRATA_HIP(launch_copy((const void*)src, (void*)dst, bytes, c->stream));
    return 0;
}

int strata_read_kernel(strata_ctx* c, uint64_t src, uint64_t bytes, uint64_t sink) {
    if (check_ctx(c)) return -1;
    if (bytes % 16) return set_error("read_kernel: bytes must be a multiple of 16");
    if (!sink) return set_error("read_kernel: null sink (256 bytes)");
    STRATA_HIP(launch_read((const void*)src, bytes, (uint32_t*)sink, c->stream));
    return 0;
}

int strata_event_destroy(void* ev) {
    STRATA_HIP(hipEventDestroy((hipEvent_t)ev));
    return 0;
}

}  // extern "C"
