// Row-wise Q8/Q4 quantization of BF16 weights (the load-time half of
// OpsToolbox::linear, ops.rs:1199-1226) and the dequantization used for
// bit-exact checks.
//
// quantize follows q8.rs:91-125 / q4.rs:126-161 step for step: max|w| per
// row (exact in any order), scale = max|w| / 127 (or / 7; 1.0 for a zero
// row), code = round-half-away(w / scale) clamped to ±127 (±7), with IEEE
// division (HIP's default correctly-rounded f32 divide). Every payload byte
// of the padded row is written, so the output needs no clearing.
#include "kernels.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int quant_code(float v, float scale, float limit) {
    float q = roundf(v / scale);
    if (q != q) return 0;  // NaN: Rust's saturating `as i8` gives 0
    q = fminf(fmaxf(q, -limit), limit);
    return (int)q;
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const uint16_t *w, int rows, int cols, uint8_t *out,
                                                            size_t row_bytes) {
    __shared__ float red[kThreads / 64];
    const int row = blockIdx.x;
    const uint16_t *src = w + (size_t)row * cols;
    float m = 0.f;
    for (int c = threadIdx.x; c < cols; c += kThreads) m = fmaxf(m, fabsf(bf16_f32(src[c])));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float max_abs = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float limit = FMT == FMT_Q8 ? 127.0f : 7.0f;
    const float scale = max_abs > 0.0f ? max_abs / limit : 1.0f;
    if (threadIdx.x == 0) ((float *)out)[row] = scale;
    uint8_t *dst = out + (size_t)rows * 4 + (size_t)row * row_bytes;
    for (size_t b = threadIdx.x; b < row_bytes; b += kThreads) {
        if constexpr (FMT == FMT_Q8) {
            dst[b] = b < (size_t)cols ? (uint8_t)(int8_t)quant_code(bf16_f32(src[b]), scale, limit) : 0;
        } else {
            const size_t c0 = 2 * b, c1 = 2 * b + 1;
            int lo = c0 < (size_t)cols ? quant_code(bf16_f32(src[c0]), scale, limit) : 0;
            int hi = c1 < (size_t)cols ? quant_code(bf16_f32(src[c1]), scale, limit) : 0;
            dst[b] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
        }
    }
}

// out[r][c] = scale[r] * code[r][c]: one IEEE multiply, as dequant_value.
template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *buf, int rows, int cols, size_t row_bytes,
                                                           float *out) {
    const int row = blockIdx.x;
    const float scale = ((const float *)buf)[row];
    const uint8_t *src = buf + (size_t)rows * 4 + (size_t)row * row_bytes;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        int code;
        if constexpr (FMT == FMT_Q8) {
            code = (int8_t)src[c];
        } else {
            uint8_t byte = src[c >> 1];
            int nib = (c & 1) ? (byte >> 4) : (byte & 0xF);
            code = nib >= 8 ? nib - 16 : nib;
        }
        out[(size_t)row * cols + c] = scale * (float)code;
    }
}

}  // namespace

int launch_quantize(int fmt, const uint16_t *w, size_t rows, size_t cols, uint8_t *out, hipStream_t s) {
    if (!w || !out || rows == 0 || cols == 0) return fail("HIP backend: quantize needs a non-empty matrix.");
    if (rows > (size_t)INT32_MAX || cols > (size_t)INT32_MAX) return fail("HIP backend: quantize shape too large.");
    const size_t rb = fmt_row_bytes(fmt, cols);
    if (fmt == FMT_Q8)
        hipLaunchKernelGGL(quantize_kernel<FMT_Q8>, dim3(rows), dim3(kThreads), 0, s, w, (int)rows, (int)cols, out, rb);
    else if (fmt == FMT_Q4)
        hipLaunchKernelGGL(quantize_kernel<FMT_Q4>, dim3(rows), dim3(kThreads), 0, s, w, (int)rows, (int)cols, out, rb);
    else
        return fail("HIP backend: quantize format must be q8 or q4.");
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int launch_dequant(const WMat &w, float *out, hipStream_t s) {
    if (!w.base || !out || w.rows == 0 || w.cols == 0) return fail("HIP backend: dequant needs a non-empty matrix.");
    if (w.fmt == FMT_Q8)
        hipLaunchKernelGGL(dequant_kernel<FMT_Q8>, dim3(w.rows), dim3(kThreads), 0, s, w.base, (int)w.rows,
                           (int)w.cols, w.row_stride(), out);
    else if (w.fmt == FMT_Q4)
        hipLaunchKernelGGL(dequant_kernel<FMT_Q4>, dim3(w.rows), dim3(kThreads), 0, s, w.base, (int)w.rows,
                           (int)w.cols, w.row_stride(), out);
    else
        return fail("HIP backend: dequant format must be q8 or q4.");
    CHIP_CHECK(hipGetLastError());
    return 0;
}

}  // namespace chip
