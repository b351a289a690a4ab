// Library lifecycle, device memory and the op-level C-ABI (include/cheetah_hip.h).
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/cheetah_hip.h"
#include "kernels.hpp"

namespace chip {

// Scratch of cheetah_hip_attention_noalloc: the split partials of one call
// (rows * q_heads * splits * (head_dim + 2) floats), at most 48 MiB, held by
// every device the library runs on until the process ends. Host code never
// passes `scratch` itself to a kernel (on the host it names a stand-in, not
// device memory): it uses the device address hipGetSymbolAddress returned at
// cheetah_hip_init, kept per device in g_scratch.
constexpr size_t kNoAllocScratchFloats = (size_t)12 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
float *g_scratch[kMaxDevices] = {};
thread_local std::string g_error;
std::mutex g_mutex;
bool g_ready = false;
int g_device = -1;
hipStream_t g_stream = nullptr;
std::string g_name = "hip-gfx950";
size_t g_max_lds = 65536;
int g_cus = 256;
size_t g_lds_per_cu = 160 * 1024;
}  // namespace

size_t device_max_lds() { return g_max_lds; }
int device_cus() { return g_cus; }
size_t device_lds_per_cu() { return g_lds_per_cu; }

void set_error(const std::string &message) { g_error = message; }
const char *last_error() { return g_error.c_str(); }
hipStream_t lib_stream() { return g_stream; }

int ensure_ready() {
    if (!g_ready) return fail("HIP backend: not initialized; call cheetah_hip_init first.");
    CHIP_CHECK(hipSetDevice(g_device));
    return 0;
}

}  // namespace chip

using namespace chip;

extern "C" {

int cheetah_hip_init(int device) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_ready) {
        if (device == g_device) return 0;
        return fail("HIP backend: already initialized on device " + std::to_string(g_device) + ".");
    }
    int count = 0;
    CHIP_CHECK(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return fail("HIP backend: device " + std::to_string(device) + " not present (" + std::to_string(count) +
                    " visible).");
    hipDeviceProp_t prop;
    CHIP_CHECK(hipGetDeviceProperties(&prop, device));
    const std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail("HIP backend: device " + std::to_string(device) + " is " + arch +
                    "; this library is built for gfx950 (MI355X) only.");
    CHIP_CHECK(hipSetDevice(device));
    if (device >= kMaxDevices) return fail("HIP backend: device index above the supported 64.");
    if (!g_scratch[device]) {
        void *p = nullptr;
        CHIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail("HIP backend: no device address for the attention scratch.");
        g_scratch[device] = (float *)p;
    }
    g_max_lds = prop.sharedMemPerBlock;
    g_cus = prop.multiProcessorCount;
    if (prop.maxSharedMemoryPerMultiProcessor > 0) g_lds_per_cu = prop.maxSharedMemoryPerMultiProcessor;
    CHIP_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_device = device;
    g_name = std::string("hip-") + arch.substr(0, 6) + " (" + prop.name + ")";
    g_ready = true;
    return 0;
}

void cheetah_hip_shutdown(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_ready) return;
    (void)hipSetDevice(g_device);
    (void)hipStreamSynchronize(g_stream);
    (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    g_ready = false;
}

const char *cheetah_hip_device_name(void) { return g_name.c_str(); }
const char *cheetah_hip_last_error(void) { return last_error(); }

void *cheetah_hip_alloc(size_t bytes) {
    if (ensure_ready()) return nullptr;
    if (bytes == 0) {
        fail("HIP backend: zero-byte allocation.");
        return nullptr;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        fail(std::string("HIP backend: hipMalloc(") + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

int cheetah_hip_free(void *p) {
    CHIP_TRY(ensure_ready());
    if (!p) return 0;
    CHIP_CHECK(hipStreamSynchronize(g_stream));
    CHIP_CHECK(hipFree(p));
    return 0;
}

int cheetah_hip_upload(void *dst, const void *src, size_t bytes) {
    CHIP_TRY(ensure_ready());
    if (!dst || (!src && bytes)) return fail("HIP backend: upload with a null pointer.");
    CHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    CHIP_CHECK(hipStreamSynchronize(g_stream));
    return 0;
}

int cheetah_hip_download(void *dst, const void *src, size_t bytes) {
    CHIP_TRY(ensure_ready());
    if (!dst || (!src && bytes)) return fail("HIP backend: download with a null pointer.");
    CHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    CHIP_CHECK(hipStreamSynchronize(g_stream));
    return 0;
}

int cheetah_hip_copy(void *dst, const void *src, size_t bytes) {
    CHIP_TRY(ensure_ready());
    if (!dst || (!src && bytes)) return fail("HIP backend: copy with a null pointer.");
    CHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    CHIP_CHECK(hipStreamSynchronize(g_stream));
    return 0;
}

int cheetah_hip_synchronize(void) {
    CHIP_TRY(ensure_ready());
    CHIP_CHECK(hipStreamSynchronize(g_stream));
    return 0;
}

static int gemv_op(int fmt, const void *w, size_t rows, size_t cols, const float *x, float *y) {
    CHIP_TRY(ensure_ready());
    if (!w || !x || !y) return fail("HIP backend: gemv with a null pointer.");
    if (rows == 0 || cols == 0) return fail("HIP backend: gemv needs rows > 0 and cols > 0.");
    GemvJob j;
    j.w = WMat{fmt, (const uint8_t *)w, rows, cols};
    j.x = x;
    j.y = y;
    return launch_gemv(j, g_stream);
}

int cheetah_hip_gemv_bf16(const uint16_t *w, size_t rows, size_t cols, const float *x, float *y) {
    return gemv_op(FMT_BF16, w, rows, cols, x, y);
}
int cheetah_hip_gemv_q8(const uint8_t *w, size_t rows, size_t cols, const float *x, float *y) {
    return gemv_op(FMT_Q8, w, rows, cols, x, y);
}
int cheetah_hip_gemv_q4(const uint8_t *w, size_t rows, size_t cols, const float *x, float *y) {
    return gemv_op(FMT_Q4, w, rows, cols, x, y);
}

// Split-K scratch of the op-level GEMM (grown on demand, per thread).
static int gemm_scratch(size_t rows, size_t cols, size_t n, GemmJob &j) {
    static thread_local float *ws = nullptr;
    static thread_local size_t ws_floats = 0;
    const size_t need = gemm_split_workspace_floats(rows, cols, n, false);
    if (need > ws_floats) {
        CHIP_CHECK(hipStreamSynchronize(g_stream));
        if (ws) CHIP_CHECK(hipFree(ws));
        ws = nullptr;
        ws_floats = 0;
        CHIP_CHECK(hipMalloc(&ws, need * sizeof(float)));
        ws_floats = need;
    }
    j.ws = ws;
    j.ws_floats = ws_floats;
    // x split into BF16 halves once per call.
    static thread_local uint16_t *xs = nullptr;
    static thread_local size_t xs_elems = 0;
    const size_t elems = n * cols;
    if (elems > xs_elems) {
        CHIP_CHECK(hipStreamSynchronize(g_stream));
        if (xs) CHIP_CHECK(hipFree(xs));
        xs = nullptr;
        xs_elems = 0;
        CHIP_CHECK(hipMalloc(&xs, 2 * elems * sizeof(uint16_t) + 256));
        xs_elems = elems;
    }
    CHIP_TRY(launch_split_bf16(j.x, elems, xs, xs + (elems + 127) / 128 * 128, g_stream));
    j.xh = xs;
    j.xl = xs + (elems + 127) / 128 * 128;
    return 0;
}

static int gemm_op(int fmt, const void *w, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    CHIP_TRY(ensure_ready());
    if (!w || !x || !y) return fail("HIP backend: gemm with a null pointer.");
    if (rows == 0 || cols == 0 || n == 0) return fail("HIP backend: gemm needs rows, cols and n > 0.");
    GemmJob j;
    j.w = WMat{fmt, (const uint8_t *)w, rows, cols};
    j.x = x;
    j.n = n;
    j.y = y;
    CHIP_TRY(gemm_scratch(rows, cols, n, j));
    return launch_gemm(j, g_stream);
}

int cheetah_hip_gemm_bf16(const uint16_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    return gemm_op(FMT_BF16, w, rows, cols, x, n, y);
}
int cheetah_hip_gemm_q8(const uint8_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    return gemm_op(FMT_Q8, w, rows, cols, x, n, y);
}
int cheetah_hip_gemm_q4(const uint8_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    return gemm_op(FMT_Q4, w, rows, cols, x, n, y);
}

size_t cheetah_hip_q8_buffer_bytes(size_t rows, size_t cols) { return fmt_buffer_bytes(FMT_Q8, rows, cols); }
size_t cheetah_hip_q4_buffer_bytes(size_t rows, size_t cols) { return fmt_buffer_bytes(FMT_Q4, rows, cols); }

static int quantize_op(int fmt, const uint16_t *w, size_t rows, size_t cols, uint8_t *out, size_t out_len) {
    CHIP_TRY(ensure_ready());
    if (!w || !out) return fail("HIP backend: quantize with a null pointer.");
    const size_t want = fmt_buffer_bytes(fmt, rows, cols);
    if (out_len != want)
        return fail(std::string(fmt == FMT_Q8 ? "Q8" : "Q4") + " quantization expected a " + std::to_string(want) +
                    "-byte buffer, found " + std::to_string(out_len) + ".");
    return launch_quantize(fmt, w, rows, cols, out, g_stream);
}

int cheetah_hip_quantize_q8(const uint16_t *w, size_t rows, size_t cols, uint8_t *out, size_t out_len) {
    return quantize_op(FMT_Q8, w, rows, cols, out, out_len);
}
int cheetah_hip_quantize_q4(const uint16_t *w, size_t rows, size_t cols, uint8_t *out, size_t out_len) {
    return quantize_op(FMT_Q4, w, rows, cols, out, out_len);
}

int cheetah_hip_dequant_q8(const uint8_t *w, size_t rows, size_t cols, float *out) {
    CHIP_TRY(ensure_ready());
    return launch_dequant(WMat{FMT_Q8, w, rows, cols}, out, g_stream);
}
int cheetah_hip_dequant_q4(const uint8_t *w, size_t rows, size_t cols, float *out) {
    CHIP_TRY(ensure_ready());
    return launch_dequant(WMat{FMT_Q4, w, rows, cols}, out, g_stream);
}

static int attention_op(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows, size_t offset,
                        float *out);

// Argument checks of the attention entry points, made before any device call
// (the split count below divides by kv_heads).
static int check_attention_args(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                                const float *out) {
    if (!q || !kv || !out) return fail("HIP backend: attention with a null pointer.");
    if (rows == 0) return fail("HIP backend: attention needs at least one query row.");
    if (kv->kv_heads == 0 || q_heads == 0 || q_heads % kv->kv_heads)
        return fail("HIP backend: q_heads must be a multiple of kv_heads.");
    if (kv->head_dim == 0 || kv->page_size == 0)
        return fail("HIP backend: attention needs a non-zero head_dim and page size.");
    return 0;
}

int cheetah_hip_attention(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                          size_t offset, float *out) {
    CHIP_TRY(check_attention_args(q, kv, q_heads, rows, out));
    CHIP_TRY(ensure_ready());
    return attention_op(q, kv, q_heads, rows, offset, out);
}

// The job of one attention call and the partial floats it needs.
static AttnJob attention_job(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                             size_t offset, float *out, size_t *need_floats) {
    AttnJob j;
    j.q = q;
    j.q_stride = (size_t)q_heads * kv->head_dim;
    j.out = out;
    j.k = kv->k_pages;
    j.v = kv->v_pages;
    j.g = KvGeom{kv->page_table, (int)kv->page_size, (int)kv->kv_heads, (int)kv->head_dim};
    j.q_heads = (int)q_heads;
    j.rows = rows;
    j.offset = offset;
    const size_t splits = (size_t)attention_decode_splits(offset + rows, (int)kv->kv_heads, rows, false);
    j.splits = (int)splits;
    j.prefill = rows > 1;
    size_t need = attention_part_floats(rows, (int)q_heads, (int)splits, (int)kv->head_dim);
    if (j.prefill && attention_prefill_on_mfma(j.g, (int)q_heads))
        need = std::max(need, attention_part_floats(rows, (int)q_heads, attention_prefill_splits(offset + rows, j.span),
                                                    (int)kv->head_dim));
    *need_floats = need;
    return j;
}

static int attention_op(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows, size_t offset,
                        float *out) {
    CHIP_TRY(check_attention_args(q, kv, q_heads, rows, out));
    static thread_local float *part = nullptr;
    static thread_local size_t part_floats = 0;
    size_t need = 0;
    AttnJob j = attention_job(q, kv, q_heads, rows, offset, out, &need);
    if (need > part_floats) {
        CHIP_CHECK(hipStreamSynchronize(g_stream));
        if (part) CHIP_CHECK(hipFree(part));
        part = nullptr;
        part_floats = 0;
        CHIP_CHECK(hipMalloc(&part, need * sizeof(float)));
        part_floats = need;
    }
    j.part = part;
    j.part_floats = part_floats;
    return launch_attention(j, g_stream);
}

int cheetah_hip_attention_noalloc(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                                  size_t offset, float *out) {
    CHIP_TRY(check_attention_args(q, kv, q_heads, rows, out));
    CHIP_TRY(ensure_ready());
    float *part = g_scratch[g_device];
    if (!part) return fail("HIP backend: the attention scratch has no device address.");
    size_t need = 0;
    AttnJob j = attention_job(q, kv, q_heads, rows, offset, out, &need);
    if (need > kNoAllocScratchFloats)
        return fail("HIP backend: attention_noalloc needs " + std::to_string(need * sizeof(float)) +
                    " bytes of split partials; its scratch holds " +
                    std::to_string(kNoAllocScratchFloats * sizeof(float)) + ".");
    // Every partial a launch reads was written by a split of the same launch
    // first: nothing in the scratch has to start at zero.
    j.part = part;
    j.part_floats = kNoAllocScratchFloats;
    return launch_attention(j, g_stream);
}

int cheetah_hip_time_gemv(uint32_t fmt, const void *const *w, size_t nbuf, size_t rows, size_t cols,
                          const float *x, float *y, size_t iters, float *ms) {
    CHIP_TRY(ensure_ready());
    if (!w || nbuf == 0 || iters == 0 || !ms) return fail("HIP backend: time_gemv needs buffers and iterations.");
    if (fmt != FMT_BF16 && fmt != FMT_Q8 && fmt != FMT_Q4) return fail("HIP backend: unknown weight format.");
    for (size_t i = 0; i < nbuf; ++i)
        if (!w[i]) return fail("HIP backend: time_gemv with a null weight buffer.");
    GemvJob j;
    j.x = x;
    j.y = y;
    hipEvent_t e0, e1;
    CHIP_CHECK(hipEventCreate(&e0));
    CHIP_CHECK(hipEventCreate(&e1));
    for (size_t i = 0; i < nbuf; ++i) {  // warm the code path
        j.w = WMat{(int)fmt, (const uint8_t *)w[i], rows, cols};
        CHIP_TRY(launch_gemv(j, g_stream));
    }
    CHIP_CHECK(hipEventRecord(e0, g_stream));
    for (size_t i = 0; i < iters; ++i) {
        j.w = WMat{(int)fmt, (const uint8_t *)w[i % nbuf], rows, cols};
        CHIP_TRY(launch_gemv(j, g_stream));
    }
    CHIP_CHECK(hipEventRecord(e1, g_stream));
    CHIP_CHECK(hipEventSynchronize(e1));
    float total = 0.f;
    CHIP_CHECK(hipEventElapsedTime(&total, e0, e1));
    *ms = total / (float)iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

int cheetah_hip_time_gemm(uint32_t fmt, const void *const *w, size_t nbuf, size_t rows, size_t cols,
                          const float *x, size_t n, float *y, size_t iters, float *ms) {
    CHIP_TRY(ensure_ready());
    if (!w || nbuf == 0 || iters == 0 || !ms || !x || !y || n == 0)
        return fail("HIP backend: time_gemm needs buffers, rows and iterations.");
    if (fmt != FMT_BF16 && fmt != FMT_Q8 && fmt != FMT_Q4) return fail("HIP backend: unknown weight format.");
    for (size_t i = 0; i < nbuf; ++i)
        if (!w[i]) return fail("HIP backend: time_gemm with a null weight buffer.");
    GemmJob j;
    j.x = x;
    j.n = n;
    j.y = y;
    CHIP_TRY(gemm_scratch(rows, cols, n, j));
    hipEvent_t e0, e1;
    CHIP_CHECK(hipEventCreate(&e0));
    CHIP_CHECK(hipEventCreate(&e1));
    for (size_t i = 0; i < nbuf; ++i) {
        j.w = WMat{(int)fmt, (const uint8_t *)w[i], rows, cols};
        CHIP_TRY(launch_gemm(j, g_stream));
    }
    CHIP_CHECK(hipEventRecord(e0, g_stream));
    for (size_t i = 0; i < iters; ++i) {
        j.w = WMat{(int)fmt, (const uint8_t *)w[i % nbuf], rows, cols};
        // The x split is part of every GEMM call on f32 activations: timed too.
        CHIP_TRY(launch_split_bf16(x, n * cols, (uint16_t *)j.xh, (uint16_t *)j.xl, g_stream));
        CHIP_TRY(launch_gemm(j, g_stream));
    }
    CHIP_CHECK(hipEventRecord(e1, g_stream));
    CHIP_CHECK(hipEventSynchronize(e1));
    float total = 0.f;
    CHIP_CHECK(hipEventElapsedTime(&total, e0, e1));
    *ms = total / (float)iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

int cheetah_hip_time_attention(const float *q, const cheetah_hip_kv_view *views, size_t nviews, uint32_t q_heads,
                               size_t rows, size_t offset, float *out, size_t iters, float *ms) {
    CHIP_TRY(ensure_ready());
    if (!views || nviews == 0 || iters == 0 || !ms) return fail("HIP backend: time_attention needs views and iterations.");
    for (size_t i = 0; i < nviews; ++i) CHIP_TRY(attention_op(q, &views[i], q_heads, rows, offset, out));
    hipEvent_t e0, e1;
    CHIP_CHECK(hipEventCreate(&e0));
    CHIP_CHECK(hipEventCreate(&e1));
    CHIP_CHECK(hipEventRecord(e0, g_stream));
    for (size_t i = 0; i < iters; ++i) CHIP_TRY(attention_op(q, &views[i % nviews], q_heads, rows, offset, out));
    CHIP_CHECK(hipEventRecord(e1, g_stream));
    CHIP_CHECK(hipEventSynchronize(e1));
    float total = 0.f;
    CHIP_CHECK(hipEventElapsedTime(&total, e0, e1));
    *ms = total / (float)iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

}  // extern "C"
