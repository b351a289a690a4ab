// cheetah_ref_cpu — CPU oracle (test infrastructure only; see ref_cpu.h).
//
// Restates the arithmetic of the reference's native CPU backend:
//   src/chat/native/ops.rs            math kernels + OpsToolbox
//   src/chat/precision/{q8,q4}.rs     quantized layouts and quantize
//   src/chat/registrations/qwen2.rs   forward assembly (llama.rs is the same
//                                     block without biases, untied head)
// Rust never contracts `a * b + c` and folds float sums left to right, so
// this file is built with -ffp-contract=off and uses FMA only through the
// explicit intrinsics the reference itself uses (dot_row_bf16_avx2,
// dot_row_bf16_avx2_multi).
#include "ref_cpu.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_error;

int fail(const std::string &message) {
    g_error = message;
    return -1;
}

// ---------------------------------------------------------------------------
// Thread pool: the reference runs rayon over physical cores (engine.rs:859).
// Work splits only by rows / heads, so results do not depend on the count.
// ---------------------------------------------------------------------------
class Pool {
  public:
    explicit Pool(int threads) { resize(threads); }
    ~Pool() { stop(); }

    void resize(int threads) {
        stop();
        threads_ = std::max(1, threads);
        quit_ = false;
        for (int i = 1; i < threads_; ++i) workers_.emplace_back([this] { loop(); });
    }
    int threads() const { return threads_; }

    // Runs fn(i) for i in [0, n); the caller participates. Each call has its
    // own job record, so a worker still leaving an earlier job can only
    // touch that job's (exhausted) counters.
    void parallel_for(size_t n, const std::function<void(size_t)> &fn) {
        if (n == 0) return;
        if (threads_ == 1 || n == 1) {
            for (size_t i = 0; i < n; ++i) fn(i);
            return;
        }
        std::unique_lock<std::mutex> call_lock(call_mutex_);
        auto job = std::make_shared<Job>();
        job->fn = &fn;
        job->n = n;
        {
            std::lock_guard<std::mutex> lock(mutex_);
            job_ = job;
            ++generation_;
        }
        cv_.notify_all();
        run_items(*job);
        std::unique_lock<std::mutex> lock(mutex_);
        done_cv_.wait(lock, [&] { return job->done.load() == job->n; });
        job_.reset();
    }

  private:
    struct Job {
        const std::function<void(size_t)> *fn = nullptr;
        size_t n = 0;
        std::atomic<size_t> next{0}, done{0};
    };

    void run_items(Job &job) {
        for (;;) {
            const size_t i = job.next.fetch_add(1);
            if (i >= job.n) break;
            (*job.fn)(i);
            if (job.done.fetch_add(1) + 1 == job.n) {
                std::lock_guard<std::mutex> lock(mutex_);
                done_cv_.notify_all();
            }
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            std::shared_ptr<Job> job;
            {
                std::unique_lock<std::mutex> lock(mutex_);
                cv_.wait(lock, [&] { return quit_ || (generation_ != seen && job_ != nullptr); });
                if (quit_) return;
                seen = generation_;
                job = job_;
            }
            run_items(*job);
        }
    }
    void stop() {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            quit_ = true;
        }
        cv_.notify_all();
        for (auto &w : workers_) w.join();
        workers_.clear();
    }

    int threads_ = 1;
    std::vector<std::thread> workers_;
    std::mutex mutex_, call_mutex_;
    std::condition_variable cv_, done_cv_;
    std::shared_ptr<Job> job_;
    uint64_t generation_ = 0;
    bool quit_ = false;
};

int default_threads() {
    unsigned hc = std::thread::hardware_concurrency();
    return hc == 0 ? 1 : (int)hc;
}

Pool &pool() {
    static Pool p(default_threads());
    return p;
}

// ---------------------------------------------------------------------------
// Scalars.
// ---------------------------------------------------------------------------

// ops.rs:58-61 — BF16 widening is a 16-bit shift.
inline float bf16_f32(uint16_t bits) {
    uint32_t u = (uint32_t)bits << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline float load_f32(const uint8_t *p) {
    float f;
    std::memcpy(&f, p, 4);
    return f;
}

// Rust's `Iterator::sum::<f32>` is a left fold from -0.0.
constexpr float kSumInit = -0.0f;

// Sums the 8 lanes left to right (ops.rs:498-504 `horizontal_sum`,
// ops.rs:227-232 `lanes.iter().sum()`).
inline float lane_sum(__m256 v) {
    alignas(32) float lanes[8];
    _mm256_store_ps(lanes, v);
    float s = kSumInit;
    for (int i = 0; i < 8; ++i) s = s + lanes[i];
    return s;
}

// ops.rs:200-239 dot_row_bf16_avx2: 16 bf16 per step, two FMA accumulators,
// per-accumulator lane sums, then a non-FMA scalar tail.
float dot_row_bf16_avx2(const uint16_t *row, size_t cols, const float *x) {
    const size_t full = cols / 16;
    __m256 acc0 = _mm256_setzero_ps();
    __m256 acc1 = _mm256_setzero_ps();
    for (size_t c = 0; c < full; ++c) {
        __m256i w = _mm256_loadu_si256((const __m256i *)(row + c * 16));
        __m128i lo = _mm256_castsi256_si128(w);
        __m128i hi = _mm256_extracti128_si256(w, 1);
        __m256 f_lo = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(lo), 16));
        __m256 f_hi = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(hi), 16));
        __m256 x0 = _mm256_loadu_ps(x + c * 16);
        __m256 x1 = _mm256_loadu_ps(x + c * 16 + 8);
        acc0 = _mm256_fmadd_ps(f_lo, x0, acc0);
        acc1 = _mm256_fmadd_ps(f_hi, x1, acc1);
    }
    float total = lane_sum(acc0) + lane_sum(acc1);
    float tail_total = 0.0f;
    for (size_t i = full * 16; i < cols; ++i) tail_total = tail_total + bf16_f32(row[i]) * x[i];
    return total + tail_total;
}

// ops.rs:136-150 dot_f32: 8 lane accumulators (no FMA), lane sum, scalar tail.
float dot_f32(const float *a, const float *b, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t chunks = n / 8;
    for (size_t c = 0; c < chunks; ++c)
        for (int lane = 0; lane < 8; ++lane) acc[lane] = acc[lane] + a[c * 8 + lane] * b[c * 8 + lane];
    float sum = kSumInit;
    for (int lane = 0; lane < 8; ++lane) sum = sum + acc[lane];
    for (size_t i = chunks * 8; i < n; ++i) sum = sum + a[i] * b[i];
    return sum;
}

constexpr size_t kGemvChunkRows = 128;  // ops.rs:51
constexpr size_t kGemmBlockRows = 64;   // ops.rs:283
constexpr size_t kGemmTokenGroup = 4;   // ops.rs:286
constexpr size_t kAttentionParallelMinCache = 384;  // ops.rs:289

// Row-chunked parallel driver shared by gemv / gemv_q8 / gemv_q4
// (ops.rs:261-277, 566-576, 620-630).
template <class RowFn>
void rows_parallel(size_t rows, float *y, RowFn dot_row) {
    if (rows <= kGemvChunkRows) {
        for (size_t r = 0; r < rows; ++r) y[r] = dot_row(r);
        return;
    }
    size_t chunks = (rows + kGemvChunkRows - 1) / kGemvChunkRows;
    pool().parallel_for(chunks, [&](size_t chunk) {
        size_t start = chunk * kGemvChunkRows;
        size_t end = std::min(rows, start + kGemvChunkRows);
        for (size_t r = start; r < end; ++r) y[r] = dot_row(r);
    });
}

// ops.rs:405-489 dot_row_bf16_avx2_multi: one weight row against up to four
// token rows; per token the same accumulation as dot_row_bf16_avx2.
void dot_row_bf16_avx2_multi(const uint16_t *row, size_t cols, const float *x,
                             size_t token_start, size_t token_count, float *out) {
    const size_t full = cols / 16;
    __m256 a00 = _mm256_setzero_ps(), a01 = _mm256_setzero_ps();
    __m256 a10 = _mm256_setzero_ps(), a11 = _mm256_setzero_ps();
    __m256 a20 = _mm256_setzero_ps(), a21 = _mm256_setzero_ps();
    __m256 a30 = _mm256_setzero_ps(), a31 = _mm256_setzero_ps();
    const float *b0 = x + token_start * cols;
    const float *b1 = token_count > 1 ? x + (token_start + 1) * cols : b0;
    const float *b2 = token_count > 2 ? x + (token_start + 2) * cols : b0;
    const float *b3 = token_count > 3 ? x + (token_start + 3) * cols : b0;
    for (size_t c = 0; c < full; ++c) {
        __m256i w = _mm256_loadu_si256((const __m256i *)(row + c * 16));
        __m128i lo = _mm256_castsi256_si128(w);
        __m128i hi = _mm256_extracti128_si256(w, 1);
        __m256 f_lo = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(lo), 16));
        __m256 f_hi = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(hi), 16));
        size_t base = c * 16;
        a00 = _mm256_fmadd_ps(f_lo, _mm256_loadu_ps(b0 + base), a00);
        a01 = _mm256_fmadd_ps(f_hi, _mm256_loadu_ps(b0 + base + 8), a01);
        a10 = _mm256_fmadd_ps(f_lo, _mm256_loadu_ps(b1 + base), a10);
        a11 = _mm256_fmadd_ps(f_hi, _mm256_loadu_ps(b1 + base + 8), a11);
        a20 = _mm256_fmadd_ps(f_lo, _mm256_loadu_ps(b2 + base), a20);
        a21 = _mm256_fmadd_ps(f_hi, _mm256_loadu_ps(b2 + base + 8), a21);
        a30 = _mm256_fmadd_ps(f_lo, _mm256_loadu_ps(b3 + base), a30);
        a31 = _mm256_fmadd_ps(f_hi, _mm256_loadu_ps(b3 + base + 8), a31);
    }
    __m256 accs[4][2] = {{a00, a01}, {a10, a11}, {a20, a21}, {a30, a31}};
    for (size_t t = 0; t < token_count; ++t) {
        const float *xr = x + (token_start + t) * cols;
        float tail_total = 0.0f;
        for (size_t i = full * 16; i < cols; ++i) tail_total = tail_total + bf16_f32(row[i]) * xr[i];
        out[t] = lane_sum(accs[t][0]) + lane_sum(accs[t][1]) + tail_total;
    }
}

// ops.rs:585-630 nibble decode (q4.rs:59-66).
inline int q4_code(uint8_t byte, size_t column) {
    uint8_t nibble = (column % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
    return nibble >= 8 ? (int)nibble - 16 : (int)nibble;
}

// Rust `(v / scale).round().clamp(lo, hi) as i8` (q8.rs:118, q4.rs:153).
inline int8_t quant_code(float value, float scale, float limit) {
    float q = std::round(value / scale);
    if (std::isnan(q)) return 0;
    q = std::min(std::max(q, -limit), limit);
    return (int8_t)q;
}

}  // namespace

// ===========================================================================
// Math kernels.
// ===========================================================================
extern "C" {

const char *ref_last_error(void) { return g_error.c_str(); }

void ref_set_threads(int threads) { pool().resize(threads <= 0 ? default_threads() : threads); }
int ref_get_threads(void) { return pool().threads(); }

// ops.rs:246-278 gemv (BF16 through the AVX2 fused dot, F32 through dot_f32).
void ref_gemv(const void *weight, int dtype, size_t rows, size_t cols, const float *x, float *y) {
    if (dtype == 1) {
        const uint16_t *w = (const uint16_t *)weight;
        rows_parallel(rows, y, [&](size_t r) { return dot_row_bf16_avx2(w + r * cols, cols, x); });
    } else {
        const float *w = (const float *)weight;
        rows_parallel(rows, y, [&](size_t r) { return dot_f32(w + r * cols, x, cols); });
    }
}

// ops.rs:308-354 gemm + gemm_row_block (364-386): 64-row blocks in parallel,
// 4-token groups per block; bit-identical to per-token gemv (ops.rs:1727).
void ref_gemm_bf16(const uint16_t *weight, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    if (n == 1) {
        ref_gemv(weight, 1, rows, cols, x, y);
        return;
    }
    std::vector<float> y_t(rows * n);
    size_t block_rows = std::min(kGemmBlockRows, rows);
    size_t blocks = (rows + block_rows - 1) / block_rows;
    auto run_block = [&](size_t b) {
        size_t row_start = b * block_rows;
        size_t rows_in_block = std::min(block_rows, rows - row_start);
        float *out = y_t.data() + row_start * n;
        for (size_t ts = 0; ts < n; ts += kGemmTokenGroup) {
            size_t count = std::min(kGemmTokenGroup, n - ts);
            for (size_t i = 0; i < rows_in_block; ++i) {
                size_t row = row_start + i;
                dot_row_bf16_avx2_multi(weight + row * cols, cols, x, ts, count, out + i * n + ts);
            }
        }
    };
    if (rows <= block_rows) run_block(0);
    else pool().parallel_for(blocks, run_block);
    for (size_t r = 0; r < rows; ++r)
        for (size_t t = 0; t < n; ++t) y[t * rows + r] = y_t[r * n + t];
}

size_t ref_q4_row_stride(size_t cols) { return ((cols + 1 + 1) / 2 + 3) / 4 * 4; }

size_t ref_q8_buffer_bytes(size_t rows, size_t cols) { return rows * 4 + rows * ((cols + 3) / 4 * 4); }
size_t ref_q4_buffer_bytes(size_t rows, size_t cols) { return rows * 4 + rows * ref_q4_row_stride(cols); }

// ops.rs:544-577 gemv_q8: sum += (scale * code) * x, sequential, no FMA.
void ref_gemv_q8(const uint8_t *buffer, size_t rows, size_t cols, const float *x, float *y) {
    const size_t row_bytes = (cols + 3) / 4 * 4;
    const size_t head = rows * 4;
    rows_parallel(rows, y, [&](size_t r) {
        float scale = load_f32(buffer + r * 4);
        const int8_t *codes = (const int8_t *)(buffer + head + r * row_bytes);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) sum = sum + scale * (float)codes[c] * x[c];
        return sum;
    });
}

// ops.rs:586-630 gemv_q4 with row stride q4.rs:50-52.
void ref_gemv_q4(const uint8_t *buffer, size_t rows, size_t cols, const float *x, float *y) {
    const size_t row_bytes = ref_q4_row_stride(cols);
    const size_t head = rows * 4;
    rows_parallel(rows, y, [&](size_t r) {
        float scale = load_f32(buffer + r * 4);
        const uint8_t *row = buffer + head + r * row_bytes;
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) sum = sum + scale * (float)q4_code(row[c / 2], c) * x[c];
        return sum;
    });
}

}  // extern "C"

namespace {

// Per-token gemv_q8 / gemv_q4 (ops.rs:544-630; the reference's linear_batch
// runs one gemv per token for quantized units, ops.rs:1244-1326) evaluated
// for many tokens at once. Vector lanes hold different tokens; each token's
// sum is still the sequential fold over columns from 0.0, with
// w = scale * code rounded once, then w * x and the add rounded separately,
// so every output is bit-identical to ref_gemv_q* on that token alone.
template <int FMT>
void gemm_quant_tokens(const uint8_t *buffer, size_t rows, size_t cols, const float *x, size_t n, float *y) {
    constexpr size_t TG = 16;  // tokens per group (two AVX2 vectors)
    constexpr size_t RB = 4;   // weight rows per block
    const size_t row_bytes = FMT == 4 ? (cols + 3) / 4 * 4 : ref_q4_row_stride(cols);
    const size_t head = rows * 4;
    const size_t groups = (n + TG - 1) / TG;
    std::vector<float> xt(groups * cols * TG, 0.0f);  // [group][col][TG]
    for (size_t t = 0; t < n; ++t)
        for (size_t c = 0; c < cols; ++c) xt[(t / TG) * cols * TG + c * TG + t % TG] = x[t * cols + c];
    const size_t blocks = (rows + RB - 1) / RB;
    pool().parallel_for(blocks, [&](size_t b) {
        const size_t r0 = b * RB, nr = std::min(RB, rows - r0);
        std::vector<float> w(RB * cols, 0.0f);
        for (size_t i = 0; i < nr; ++i) {
            const float scale = load_f32(buffer + (r0 + i) * 4);
            const uint8_t *row = buffer + head + (r0 + i) * row_bytes;
            for (size_t c = 0; c < cols; ++c) {
                const float code = FMT == 4 ? (float)(int8_t)row[c] : (float)q4_code(row[c / 2], c);
                w[i * cols + c] = scale * code;
            }
        }
        alignas(32) float lanes[TG];
        for (size_t g = 0; g < groups; ++g) {
            __m256 acc[RB][2];
            for (size_t i = 0; i < RB; ++i) acc[i][0] = acc[i][1] = _mm256_setzero_ps();
            const float *xg = xt.data() + g * cols * TG;
            for (size_t c = 0; c < cols; ++c) {
                const __m256 x0 = _mm256_loadu_ps(xg + c * TG), x1 = _mm256_loadu_ps(xg + c * TG + 8);
                for (size_t i = 0; i < RB; ++i) {
                    const __m256 wv = _mm256_broadcast_ss(&w[i * cols + c]);
                    acc[i][0] = _mm256_add_ps(acc[i][0], _mm256_mul_ps(wv, x0));
                    acc[i][1] = _mm256_add_ps(acc[i][1], _mm256_mul_ps(wv, x1));
                }
            }
            for (size_t i = 0; i < nr; ++i) {
                _mm256_store_ps(lanes, acc[i][0]);
                _mm256_store_ps(lanes + 8, acc[i][1]);
                for (size_t t = 0; t < TG && g * TG + t < n; ++t) y[(g * TG + t) * rows + r0 + i] = lanes[t];
            }
        }
    });
}

}  // namespace

extern "C" {

// n tokens through gemv_q8 (fmt 4) or gemv_q4 (fmt 5), bit-identical to n
// separate ref_gemv_q* calls; y is [n][rows].
void ref_gemm_quant(const uint8_t *buffer, uint32_t fmt, size_t rows, size_t cols, const float *x, size_t n,
                    float *y) {
    if (n == 1) {
        if (fmt == 4) ref_gemv_q8(buffer, rows, cols, x, y);
        else ref_gemv_q4(buffer, rows, cols, x, y);
        return;
    }
    if (fmt == 4) gemm_quant_tokens<4>(buffer, rows, cols, x, n, y);
    else gemm_quant_tokens<5>(buffer, rows, cols, x, n, y);
}

// q8.rs:91-125 quantize: scale = max|w| / 127 (1.0 for a zero row).
int ref_quantize_q8(const float *values, size_t rows, size_t cols, uint8_t *out, size_t out_len) {
    if (out_len != ref_q8_buffer_bytes(rows, cols))
        return fail("Q8 quantization output buffer has the wrong length.");
    std::memset(out, 0, out_len);
    const size_t row_bytes = (cols + 3) / 4 * 4;
    // Rows are independent, so they are quantized in parallel blocks.
    pool().parallel_for((rows + 63) / 64, [&](size_t blk) {
        for (size_t r = blk * 64; r < std::min(rows, blk * 64 + 64); ++r) {
            const float *v = values + r * cols;
            float max_abs = 0.0f;
            for (size_t c = 0; c < cols; ++c) max_abs = std::fmax(max_abs, std::fabs(v[c]));
            float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
            std::memcpy(out + r * 4, &scale, 4);
            for (size_t c = 0; c < cols; ++c)
                out[rows * 4 + r * row_bytes + c] = (uint8_t)quant_code(v[c], scale, 127.0f);
        }
    });
    return 0;
}

// q4.rs:126-161 quantize: scale = max|w| / 7, low nibble = even column.
int ref_quantize_q4(const float *values, size_t rows, size_t cols, uint8_t *out, size_t out_len) {
    if (out_len != ref_q4_buffer_bytes(rows, cols))
        return fail("Q4 quantization output buffer has the wrong length.");
    std::memset(out, 0, out_len);
    const size_t row_bytes = ref_q4_row_stride(cols);
    pool().parallel_for((rows + 63) / 64, [&](size_t blk) {
        for (size_t r = blk * 64; r < std::min(rows, blk * 64 + 64); ++r) {
            const float *v = values + r * cols;
            float max_abs = 0.0f;
            for (size_t c = 0; c < cols; ++c) max_abs = std::fmax(max_abs, std::fabs(v[c]));
            float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
            std::memcpy(out + r * 4, &scale, 4);
            for (size_t c = 0; c < cols; ++c) {
                int8_t q = quant_code(v[c], scale, 7.0f);
                out[rows * 4 + r * row_bytes + c / 2] |= (uint8_t)(((uint8_t)q & 0x0F) << ((c % 2) * 4));
            }
        }
    });
    return 0;
}

// q8.rs Q8Matrix::dequant_value: scale * code.
float ref_q8_dequant_value(const uint8_t *buffer, size_t rows, size_t cols, size_t row, size_t col) {
    const size_t row_bytes = (cols + 3) / 4 * 4;
    float scale = load_f32(buffer + row * 4);
    return scale * (float)(int8_t)buffer[rows * 4 + row * row_bytes + col];
}

// q4.rs:101-110 Q4Matrix::dequant_value.
float ref_q4_dequant_value(const uint8_t *buffer, size_t rows, size_t cols, size_t row, size_t col) {
    float scale = load_f32(buffer + row * 4);
    uint8_t byte = buffer[rows * 4 + row * ref_q4_row_stride(cols) + col / 2];
    return scale * (float)q4_code(byte, col);
}

// ops.rs:646-652 rmsnorm: sequential sum of squares, x *= inv * w.
void ref_rmsnorm(float *x, size_t n, const uint16_t *weight_bf16, float eps) {
    float ss = kSumInit;
    for (size_t i = 0; i < n; ++i) ss = ss + x[i] * x[i];
    float mean_square = ss / (float)n;
    float inv = 1.0f / std::sqrt(mean_square + eps);
    for (size_t i = 0; i < n; ++i) x[i] = x[i] * (inv * bf16_f32(weight_bf16[i]));
}

// ops.rs:693-714 rope_in_place (rotate-half, libm powf/sinf/cosf).
void ref_rope_in_place(float *values, size_t heads, size_t head_dim, size_t position, float theta) {
    const size_t half = head_dim / 2;
    for (size_t h = 0; h < heads; ++h) {
        float *base = values + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            float freq = powf(theta, -2.0f * (float)i / (float)head_dim);
            float angle = (float)position * freq;
            float s = sinf(angle), c = cosf(angle);
            float a = base[i], b = base[half + i];
            base[i] = a * c - b * s;
            base[half + i] = b * c + a * s;
        }
    }
}

// ops.rs:721-740 rope_heads: leading rotary_dim dims of every head.
void ref_rope_heads(float *values, size_t heads, size_t head_dim, size_t rotary_dim, size_t position,
                    float theta) {
    for (size_t h = 0; h < heads; ++h) ref_rope_in_place(values + h * head_dim, 1, rotary_dim, position, theta);
}

// ops.rs:743-747 silu_multiply: g = g * (u / (1 + exp(-g))).
void ref_silu_multiply(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; ++i) gate[i] = gate[i] * (up[i] / (1.0f + expf(-gate[i])));
}

// ops.rs:770-781 softmax.
void ref_softmax(float *scores, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = std::fmax(max, scores[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        scores[i] = expf(scores[i] - max);
        sum = sum + scores[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) scores[i] = scores[i] * inv;
}

}  // extern "C"

namespace {

// ops.rs:1424-1467 attention_head.
void attention_head(const float *keys, const float *values, const float *q, size_t cache_len,
                    size_t window_start, size_t kv_dim, size_t head_group, size_t head_dim, float scale,
                    size_t head, float *out_head) {
    size_t kv_head = head / head_group;
    const float *qh = q + head * head_dim;
    size_t kv_base = kv_head * head_dim;
    std::vector<float> scores(cache_len, -INFINITY);
    for (size_t pos = window_start; pos < cache_len; ++pos) {
        const float *k = keys + pos * kv_dim + kv_base;
        float s = kSumInit;
        for (size_t d = 0; d < head_dim; ++d) s = s + k[d] * qh[d];
        scores[pos] = s * scale;
    }
    ref_softmax(scores.data(), cache_len);
    for (size_t d = 0; d < head_dim; ++d) out_head[d] = 0.0f;
    for (size_t pos = window_start; pos < cache_len; ++pos) {
        float w = scores[pos];
        if (w == 0.0f) continue;
        const float *v = values + pos * kv_dim + kv_base;
        for (size_t d = 0; d < head_dim; ++d) out_head[d] = out_head[d] + w * v[d];
    }
}

}  // namespace

extern "C" void ref_attention(const float *keys, const float *values, size_t cache_len, const float *q,
                              float *out, size_t q_heads, size_t kv_heads, size_t head_dim, size_t position,
                              size_t sliding_window) {
    // ops.rs:1357-1402.
    size_t kv_dim = kv_heads * head_dim;
    size_t head_group = q_heads / kv_heads;
    float scale = 1.0f / std::sqrt((float)head_dim);
    size_t window_start = sliding_window == 0 ? 0 : ((position + 1) > sliding_window ? position + 1 - sliding_window : 0);
    window_start = std::min(window_start, cache_len > 0 ? cache_len - 1 : 0);
    auto run = [&](size_t h) {
        attention_head(keys, values, q, cache_len, window_start, kv_dim, head_group, head_dim, scale, h,
                       out + h * head_dim);
    };
    if (q_heads > 1 && cache_len >= kAttentionParallelMinCache) pool().parallel_for(q_heads, run);
    else
        for (size_t h = 0; h < q_heads; ++h) run(h);
}

namespace {

// Keys regrouped as [kv_head][block of 8 positions][head_dim][8] (the last
// block zero-padded), so that 8 positions' scores sit in one vector's lanes.
size_t block_keys(const float *keys, size_t len, size_t kv_heads, size_t hd, std::vector<float> &kt) {
    const size_t blocks = (len + 7) / 8;
    kt.assign(kv_heads * blocks * hd * 8, 0.0f);
    const size_t kv_dim = kv_heads * hd, span = 64;
    const size_t items = (blocks + span - 1) / span;
    pool().parallel_for(kv_heads * items, [&](size_t it) {
        const size_t h = it / items, b0 = (it % items) * span, b1 = std::min(blocks, b0 + span);
        for (size_t b = b0; b < b1; ++b) {
            float *dst = kt.data() + (h * blocks + b) * hd * 8;
            for (size_t j = 0; j < 8 && b * 8 + j < len; ++j) {
                const float *src = keys + (b * 8 + j) * kv_dim + h * hd;
                for (size_t d = 0; d < hd; ++d) dst[d * 8 + j] = src[d];
            }
        }
    });
    return blocks;
}

constexpr size_t kTile = 8;  // (row, head) pairs of one KV head per tile

// attention_head (ops.rs:1424-1467) for up to 8 (row, head) pairs that share
// a KV head, so each key block and value row is loaded once per tile. Per
// pair the arithmetic is the scalar code's: every score is the sequential
// fold over head_dim from -0.0 (product, then add, each rounded) times
// 1/sqrt(hd); the same softmax; every output dim the sequential fold over
// positions of w * v from 0.0. Positions a pair does not see get w = 0,
// whose product +-0 leaves a finite fold unchanged, like the reference's
// `w == 0` skip.
struct TilePair {
    const float *q;
    float *out;
    size_t len, window_start;
};

void attention_tile(const float *kt_head, const float *values, const TilePair *pairs, size_t np, size_t kv_dim,
                    size_t kv_base, size_t hd, float scale) {
    size_t max_len = 0, min_ws = SIZE_MAX;
    for (size_t j = 0; j < np; ++j) {
        max_len = std::max(max_len, pairs[j].len);
        min_ws = std::min(min_ws, pairs[j].window_start);
    }
    thread_local std::vector<float> scores, zeros;
    scores.assign(kTile * max_len, -INFINITY);
    zeros.assign(hd, 0.0f);
    const float *qs[kTile];
    for (size_t j = 0; j < kTile; ++j) qs[j] = j < np ? pairs[j].q : zeros.data();
    alignas(32) float lanes[kTile][8];
    for (size_t b = min_ws / 8; b < (max_len + 7) / 8; ++b) {
        __m256 acc[kTile];
        for (size_t j = 0; j < kTile; ++j) acc[j] = _mm256_set1_ps(kSumInit);
        const float *k = kt_head + b * hd * 8;
        for (size_t d = 0; d < hd; ++d) {
            const __m256 kv = _mm256_loadu_ps(k + d * 8);
            for (size_t j = 0; j < kTile; ++j)
                acc[j] = _mm256_add_ps(acc[j], _mm256_mul_ps(kv, _mm256_broadcast_ss(qs[j] + d)));
        }
        for (size_t j = 0; j < kTile; ++j) _mm256_store_ps(lanes[j], acc[j]);
        for (size_t j = 0; j < np; ++j)
            for (size_t l = 0; l < 8; ++l) {
                const size_t pos = b * 8 + l;
                if (pos >= pairs[j].window_start && pos < pairs[j].len)
                    scores[j * max_len + pos] = lanes[j][l] * scale;
            }
    }
    for (size_t j = 0; j < np; ++j) {
        float *sj = scores.data() + j * max_len;
        ref_softmax(sj, pairs[j].len);
        for (size_t pos = pairs[j].len; pos < max_len; ++pos) sj[pos] = 0.0f;
    }
    for (size_t j = np; j < kTile; ++j)
        for (size_t pos = 0; pos < max_len; ++pos) scores[j * max_len + pos] = 0.0f;
    for (size_t dc = 0; dc < hd; dc += 8) {
        __m256 acc[kTile];
        for (size_t j = 0; j < kTile; ++j) acc[j] = _mm256_setzero_ps();
        for (size_t pos = min_ws; pos < max_len; ++pos) {
            const __m256 v = _mm256_loadu_ps(values + pos * kv_dim + kv_base + dc);
            for (size_t j = 0; j < kTile; ++j)
                acc[j] = _mm256_add_ps(acc[j], _mm256_mul_ps(_mm256_broadcast_ss(&scores[j * max_len + pos]), v));
        }
        for (size_t j = 0; j < np; ++j) _mm256_storeu_ps(pairs[j].out + dc, acc[j]);
    }
}

}  // namespace

extern "C" void ref_attention_rows(const float *keys, const float *values, size_t offset, size_t rows,
                                   const float *q, float *out, size_t q_heads, size_t kv_heads, size_t head_dim,
                                   size_t sliding_window) {
    if (rows == 0) return;
    const size_t kv_dim = kv_heads * head_dim, group = q_heads / kv_heads, qd = q_heads * head_dim;
    if (head_dim % 8 != 0) {  // the tiles work in 8-dim slices; other widths take the per-row code
        for (size_t r = 0; r < rows; ++r)
            ref_attention(keys, values, offset + r + 1, q + r * qd, out + r * qd, q_heads, kv_heads, head_dim,
                          offset + r, sliding_window);
        return;
    }
    std::vector<float> kt;
    const size_t blocks = block_keys(keys, offset + rows, kv_heads, head_dim, kt);
    const float scale = 1.0f / std::sqrt((float)head_dim);
    const size_t pairs_per_head = rows * group, tiles = (pairs_per_head + kTile - 1) / kTile;
    pool().parallel_for(kv_heads * tiles, [&](size_t it) {
        const size_t kvh = it / tiles, p0 = (it % tiles) * kTile;
        const size_t np = std::min(kTile, pairs_per_head - p0);
        TilePair pairs[kTile];
        for (size_t j = 0; j < np; ++j) {
            const size_t r = (p0 + j) / group, h = kvh * group + (p0 + j) % group;
            const size_t position = offset + r, len = position + 1;
            size_t ws = sliding_window == 0 ? 0 : (len > sliding_window ? len - sliding_window : 0);
            pairs[j] = TilePair{q + r * qd + h * head_dim, out + r * qd + h * head_dim, len, std::min(ws, len - 1)};
        }
        attention_tile(kt.data() + kvh * blocks * head_dim * 8, values, pairs, np, kv_dim, kvh * head_dim,
                       head_dim, scale);
    });
}

// ===========================================================================
// Model: OpsToolbox state + the qwen2/llama forward assembly.
// ===========================================================================
namespace {

struct Unit {
    const uint8_t *bytes = nullptr;
    size_t nbytes = 0;
    int dtype = 1;
    std::vector<uint64_t> shape;
};

struct Weights {
    ref_config cfg{};
    std::unordered_map<std::string, Unit> units;
};

}  // namespace

struct ref_snapshot {
    size_t positions = 0;
    std::vector<std::vector<float>> kv_k, kv_v;
};

struct ref_model {
    std::shared_ptr<Weights> w;
    uint32_t quant_format = 0;
    int kv_bf16 = 0;
    std::vector<std::vector<float>> kv_k, kv_v;
    // Quantized linear buffers, filled at first use (ops.rs:1199-1226); a
    // clone starts without them (ops.rs:1017-1029).
    std::unordered_map<std::string, std::vector<uint8_t>> quant;
    // Scratch (ops.rs Scratch / ChunkScratch).
    std::vector<float> hidden, normed, q, k, v, attn_out, proj, gate, up, mlp;

    const ref_config &cfg() const { return w->cfg; }
};

namespace {

const Unit *find_unit(const ref_model *m, const std::string &id) {
    auto it = m->w->units.find(id);
    return it == m->w->units.end() ? nullptr : &it->second;
}

float scalar_at(const Unit &u, size_t index) {
    if (u.dtype == 1) {
        uint16_t bits;
        std::memcpy(&bits, u.bytes + 2 * index, 2);
        return bf16_f32(bits);
    }
    return load_f32(u.bytes + 4 * index);
}

// The BF16-KV mode's cache element (the reference's cache is f32,
// ops.rs:995-999): f32 -> BF16 round to nearest, ties to even, on the bit
// pattern (finite inputs; the overflow past the largest BF16 gives inf).
inline float round_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" void ref_round_bf16(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = round_bf16(in[i]);
}

namespace {

// ops.rs:1102-1106 rmsnorm against `{unit}.weight`.
int norm_rows(ref_model *m, const std::string &unit, float *x, size_t rows) {
    const Unit *u = find_unit(m, unit + ".weight");
    if (!u) return fail("Native backend: missing unit '" + unit + ".weight'.");
    size_t h = m->cfg().hidden_size;
    for (size_t r = 0; r < rows; ++r) {
        float *row = x + r * h;
        float ss = kSumInit;
        for (size_t i = 0; i < h; ++i) ss = ss + row[i] * row[i];
        float inv = 1.0f / std::sqrt(ss / (float)h + m->cfg().rms_eps);
        for (size_t i = 0; i < h; ++i) row[i] = row[i] * (inv * scalar_at(*u, i));
    }
    return 0;
}

// ops.rs:1156-1166 add_bias: a no-op when the unit is absent.
void add_bias_rows(ref_model *m, const std::string &unit, float *x, size_t rows, size_t width) {
    const Unit *u = find_unit(m, unit + ".bias");
    if (!u || u->nbytes == 0) return;
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < width; ++i) x[r * width + i] = x[r * width + i] + scalar_at(*u, i);
}

// ops.rs:1180-1237 linear / 1244-1326 linear_batch.
int linear_rows(ref_model *m, const std::string &unit, size_t rows, size_t cols, const float *x, size_t n,
                float *y) {
    const Unit *u = find_unit(m, unit);
    if (!u) return fail("Native backend: missing unit '" + unit + "'.");
    if (m->quant_format == 4 || m->quant_format == 5) {
        auto it = m->quant.find(unit);
        if (it == m->quant.end()) {
            size_t count = rows * cols;
            size_t esize = u->dtype == 1 ? 2 : 4;
            if (u->nbytes != count * esize)
                return fail("Linear unit '" + unit + "' does not match its " + std::to_string(rows) + "x" +
                            std::to_string(cols) + " shape.");
            std::vector<float> values(count);
            pool().parallel_for((count + (1 << 20) - 1) >> 20, [&](size_t b) {
                for (size_t i = b << 20; i < std::min(count, (b + 1) << 20); ++i) values[i] = scalar_at(*u, i);
            });
            std::vector<uint8_t> buf(m->quant_format == 4 ? ref_q8_buffer_bytes(rows, cols)
                                                          : ref_q4_buffer_bytes(rows, cols));
            if (m->quant_format == 4) ref_quantize_q8(values.data(), rows, cols, buf.data(), buf.size());
            else ref_quantize_q4(values.data(), rows, cols, buf.data(), buf.size());
            it = m->quant.emplace(unit, std::move(buf)).first;
        }
        ref_gemm_quant(it->second.data(), m->quant_format, rows, cols, x, n, y);
        return 0;
    }
    if (u->dtype == 1) {
        if (n == 1) ref_gemv(u->bytes, 1, rows, cols, x, y);
        else ref_gemm_bf16((const uint16_t *)u->bytes, rows, cols, x, n, y);
    } else {
        for (size_t t = 0; t < n; ++t) ref_gemv(u->bytes, 0, rows, cols, x + t * cols, y + t * rows);
    }
    return 0;
}

void cache_append(ref_model *m, size_t layer, const float *k, const float *v) {
    size_t kv_dim = (size_t)m->cfg().kv_heads * m->cfg().head_dim;
    auto &kk = m->kv_k[layer];
    auto &vv = m->kv_v[layer];
    if (m->kv_bf16) {
        for (size_t i = 0; i < kv_dim; ++i) kk.push_back(round_bf16(k[i]));
        for (size_t i = 0; i < kv_dim; ++i) vv.push_back(round_bf16(v[i]));
    } else {
        kk.insert(kk.end(), k, k + kv_dim);
        vv.insert(vv.end(), v, v + kv_dim);
    }
}

// qwen2.rs:240-426 forward_layer_chunk (rows == 1 is forward_layer 430-597:
// the same arithmetic, since gemm == per-token gemv bit for bit).
int forward_layer_chunk(ref_model *m, size_t layer, size_t offset, size_t rows) {
    const ref_config &c = m->cfg();
    const size_t H = c.hidden_size, qd = (size_t)c.q_heads * c.head_dim, kvd = (size_t)c.kv_heads * c.head_dim;
    const size_t I = c.intermediate_size;
    const std::string p = "model.layers." + std::to_string(layer) + ".";
    std::memcpy(m->normed.data(), m->hidden.data(), rows * H * 4);
    if (norm_rows(m, p + "input_layernorm", m->normed.data(), rows)) return -1;
    if (linear_rows(m, p + "self_attn.q_proj.weight", qd, H, m->normed.data(), rows, m->q.data())) return -1;
    if (linear_rows(m, p + "self_attn.k_proj.weight", kvd, H, m->normed.data(), rows, m->k.data())) return -1;
    if (linear_rows(m, p + "self_attn.v_proj.weight", kvd, H, m->normed.data(), rows, m->v.data())) return -1;
    add_bias_rows(m, p + "self_attn.q_proj", m->q.data(), rows, qd);
    add_bias_rows(m, p + "self_attn.k_proj", m->k.data(), rows, kvd);
    add_bias_rows(m, p + "self_attn.v_proj", m->v.data(), rows, kvd);
    // The reference ropes, appends and attends row by row (qwen2.rs:314-343).
    // Row r reads only cache positions <= offset + r and the appended K/V do
    // not depend on attention outputs, so the rows are roped in parallel,
    // appended in order, then attended in parallel with identical results.
    pool().parallel_for(rows, [&](size_t r) {
        ref_rope_heads(m->q.data() + r * qd, c.q_heads, c.head_dim, c.rotary_dim, offset + r, c.rope_theta);
        ref_rope_heads(m->k.data() + r * kvd, c.kv_heads, c.head_dim, c.rotary_dim, offset + r, c.rope_theta);
    });
    for (size_t r = 0; r < rows; ++r) cache_append(m, layer, m->k.data() + r * kvd, m->v.data() + r * kvd);
    if (m->kv_k[layer].size() / kvd != offset + rows) return fail("KV cache length does not match the offset.");
    ref_attention_rows(m->kv_k[layer].data(), m->kv_v[layer].data(), offset, rows, m->q.data(),
                       m->attn_out.data(), c.q_heads, c.kv_heads, c.head_dim, c.sliding_window);
    if (linear_rows(m, p + "self_attn.o_proj.weight", H, qd, m->attn_out.data(), rows, m->proj.data())) return -1;
    add_bias_rows(m, p + "self_attn.o_proj", m->proj.data(), rows, H);
    for (size_t i = 0; i < rows * H; ++i) m->hidden[i] = m->hidden[i] + m->proj[i];
    std::memcpy(m->normed.data(), m->hidden.data(), rows * H * 4);
    if (norm_rows(m, p + "post_attention_layernorm", m->normed.data(), rows)) return -1;
    if (linear_rows(m, p + "mlp.gate_proj.weight", I, H, m->normed.data(), rows, m->gate.data())) return -1;
    if (linear_rows(m, p + "mlp.up_proj.weight", I, H, m->normed.data(), rows, m->up.data())) return -1;
    for (size_t r = 0; r < rows; ++r) ref_silu_multiply(m->gate.data() + r * I, m->up.data() + r * I, I);
    if (linear_rows(m, p + "mlp.down_proj.weight", H, I, m->gate.data(), rows, m->mlp.data())) return -1;
    for (size_t i = 0; i < rows * H; ++i) m->hidden[i] = m->hidden[i] + m->mlp[i];
    return 0;
}

void size_scratch(ref_model *m, size_t rows) {
    const ref_config &c = m->cfg();
    const size_t H = c.hidden_size, qd = (size_t)c.q_heads * c.head_dim, kvd = (size_t)c.kv_heads * c.head_dim;
    if (m->hidden.size() >= rows * H) return;
    m->hidden.assign(rows * H, 0.f);
    m->normed.assign(rows * H, 0.f);
    m->q.assign(rows * qd, 0.f);
    m->k.assign(rows * kvd, 0.f);
    m->v.assign(rows * kvd, 0.f);
    m->attn_out.assign(rows * qd, 0.f);
    m->proj.assign(rows * H, 0.f);
    m->gate.assign(rows * c.intermediate_size, 0.f);
    m->up.assign(rows * c.intermediate_size, 0.f);
    m->mlp.assign(rows * H, 0.f);
}

}  // namespace

extern "C" {

ref_model *ref_model_create(const ref_config *cfg, uint32_t quant_format, int kv_bf16) {
    if (!cfg || cfg->num_layers == 0 || cfg->hidden_size == 0 || cfg->q_heads == 0 || cfg->kv_heads == 0 ||
        cfg->q_heads % cfg->kv_heads != 0 || cfg->head_dim == 0 || cfg->vocab_size == 0) {
        fail("Invalid decoder configuration.");
        return nullptr;
    }
    if (quant_format != 0 && quant_format != 4 && quant_format != 5) {
        fail("Unknown quantization format.");
        return nullptr;
    }
    auto *m = new ref_model();
    m->w = std::make_shared<Weights>();
    m->w->cfg = *cfg;
    if (m->w->cfg.rotary_dim == 0) m->w->cfg.rotary_dim = cfg->head_dim;
    m->quant_format = quant_format;
    m->kv_bf16 = kv_bf16;
    m->kv_k.assign(cfg->num_layers, {});
    m->kv_v.assign(cfg->num_layers, {});
    return m;
}

int ref_model_set_unit(ref_model *m, const char *unit_id, const void *bytes, size_t nbytes, int dtype,
                       const uint64_t *shape, size_t ndim) {
    if (!m || !unit_id || (!bytes && nbytes)) return fail("Invalid unit arguments.");
    Unit u;
    u.bytes = (const uint8_t *)bytes;
    u.nbytes = nbytes;
    u.dtype = dtype;
    u.shape.assign(shape, shape + ndim);
    m->w->units[unit_id] = u;
    return 0;
}

// qwen2.rs:132-154 forward_with_chunk (+ forward_chunked 193-206,
// forward_chunk 208-234, lm_head 160-170, ops.rs:1513-1563 lm_head_into).
int ref_model_forward(ref_model *m, const uint32_t *tokens, size_t n, size_t offset, size_t chunk_rows,
                      float *logits) {
    if (!m) return fail("Native backend: no model.");
    const ref_config &c = m->cfg();
    // ops.rs:1065-1078 validate_tokens.
    if (n == 0) return fail("Native backend: empty token input.");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= c.vocab_size)
            return fail("Native backend: token id " + std::to_string(tokens[i]) +
                        " exceeds the vocabulary size " + std::to_string(c.vocab_size) + ".");
    const size_t H = c.hidden_size;
    const Unit *emb = find_unit(m, "model.embed_tokens.weight");
    if (!emb) return fail("Native backend: missing unit 'model.embed_tokens.weight'.");
    if (chunk_rows == 0) chunk_rows = 1;
    if (n == 1) chunk_rows = 1;
    std::vector<float> last(H);
    for (size_t start = 0; start < n; start += chunk_rows) {
        size_t rows = std::min(chunk_rows, n - start);
        size_scratch(m, rows);
        for (size_t r = 0; r < rows; ++r)
            for (size_t i = 0; i < H; ++i) m->hidden[r * H + i] = scalar_at(*emb, (size_t)tokens[start + r] * H + i);
        for (size_t layer = 0; layer < c.num_layers; ++layer)
            if (forward_layer_chunk(m, layer, offset + start, rows)) return -1;
        std::memcpy(last.data(), m->hidden.data() + (rows - 1) * H, H * 4);
        if (norm_rows(m, "model.norm", last.data(), 1)) return -1;
    }
    const char *head_id = c.tie_word_embeddings ? "model.embed_tokens.weight" : "lm_head.weight";
    const Unit *head = find_unit(m, head_id);
    if (!head)
        return fail(std::string("Native backend: neither tied embeddings nor a separate '") + head_id +
                    "' tensor are present.");
    const size_t esize = head->dtype == 1 ? 2 : 4;
    for (size_t start = 0; start < c.vocab_size; start += 16384) {
        size_t end = std::min<size_t>(start + 16384, c.vocab_size);
        ref_gemv(head->bytes + start * H * esize, head->dtype, end - start, H, last.data(), logits + start);
    }
    return 0;
}

void ref_model_clear_cache(ref_model *m) {
    for (auto &v : m->kv_k) v.clear();
    for (auto &v : m->kv_v) v.clear();
}

ref_model *ref_model_clone(const ref_model *src) {
    auto *m = new ref_model();
    m->w = src->w;
    m->quant_format = src->quant_format;
    m->kv_bf16 = src->kv_bf16;
    m->kv_k.assign(src->cfg().num_layers, {});
    m->kv_v.assign(src->cfg().num_layers, {});
    return m;
}

size_t ref_model_kv_len(const ref_model *m) {
    size_t kvd = (size_t)m->cfg().kv_heads * m->cfg().head_dim;
    return m->kv_k.empty() ? 0 : m->kv_k[0].size() / kvd;
}

// ops.rs:1575-1587 kv_snapshot: a full clone of every layer's f32 rows.
ref_snapshot *ref_model_kv_snapshot(const ref_model *m) {
    auto *s = new ref_snapshot();
    s->positions = ref_model_kv_len(m);
    s->kv_k = m->kv_k;
    s->kv_v = m->kv_v;
    return s;
}

// ops.rs:1593-1606 restore_kv_prefix: truncating copy of the first positions.
int ref_model_restore_kv_prefix(ref_model *m, const ref_snapshot *s, size_t positions) {
    size_t kvd = (size_t)m->cfg().kv_heads * m->cfg().head_dim;
    size_t keep = std::min(positions, s->positions) * kvd;
    for (size_t l = 0; l < m->kv_k.size(); ++l) {
        m->kv_k[l].assign(s->kv_k[l].begin(), s->kv_k[l].begin() + std::min(keep, s->kv_k[l].size()));
        m->kv_v[l].assign(s->kv_v[l].begin(), s->kv_v[l].begin() + std::min(keep, s->kv_v[l].size()));
    }
    return 1;
}

size_t ref_snapshot_positions(const ref_snapshot *s) { return s ? s->positions : 0; }
void ref_snapshot_free(ref_snapshot *s) { delete s; }
void ref_model_free(ref_model *m) { delete m; }

}  // extern "C"
