// Shared device/host helpers for the gfx950 decoder-forward kernels.
//
// Everything is built with -ffp-contract=off: a*b+c is two roundings unless
// the code writes fmaf() itself. The reference (Rust) never contracts, and
// the elementwise steps that must stay bit-identical to it (RoPE, residual
// adds, bias adds, dequantization, quantization) rely on this.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace chip {

// ---------------------------------------------------------------------------
// Error plumbing: a thread-local sentence, -1 returns (cheetah_vulkan.c-style).
// ---------------------------------------------------------------------------
void set_error(const std::string &message);
const char *last_error();

#define CHIP_CHECK(expr)                                                                      \
    do {                                                                                      \
        hipError_t chip_err_ = (expr);                                                        \
        if (chip_err_ != hipSuccess) {                                                        \
            ::chip::set_error(std::string("HIP backend: ") + #expr + " failed: " +             \
                              hipGetErrorString(chip_err_));                                  \
            return -1;                                                                        \
        }                                                                                     \
    } while (0)

#define CHIP_TRY(expr)                 \
    do {                               \
        if ((expr) != 0) return -1;    \
    } while (0)

inline int fail(const std::string &message) {
    set_error(message);
    return -1;
}

// Weight formats (codes match the reference's format ids: stored BF16 = 1,
// q8 = 4, q4 = 5; precision.rs registry).
enum WFmt : int { FMT_BF16 = 1, FMT_Q8 = 4, FMT_Q4 = 5 };

inline size_t q8_row_bytes(size_t cols) { return (cols + 3) / 4 * 4; }
inline size_t q4_row_bytes(size_t cols) { return ((cols + 2) / 2 + 3) / 4 * 4; }
inline size_t fmt_row_bytes(int fmt, size_t cols) {
    return fmt == FMT_BF16 ? cols * 2 : fmt == FMT_Q8 ? q8_row_bytes(cols) : q4_row_bytes(cols);
}
inline size_t fmt_buffer_bytes(int fmt, size_t rows, size_t cols) {
    return fmt == FMT_BF16 ? rows * cols * 2 : rows * 4 + rows * fmt_row_bytes(fmt, cols);
}

// The library stream used by the op-level entry points.
hipStream_t lib_stream();

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Device scalars.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t word) { return __uint_as_float(word & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_f32(uint16_t bits) { return __uint_as_float((uint32_t)bits << 16); }

// f32 -> BF16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Signed byte B of v as f32 in one instruction (the SDWA form the compiler
// itself emits for int8 converts; spelled out because it does not find it
// for bytes built from nibbles).
template <int B>
__device__ __forceinline__ float sbyte_f32(uint32_t v) {
    float f;
    if constexpr (B == 0) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(f) : "v"(v));
    else if constexpr (B == 1) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(f) : "v"(v));
    else if constexpr (B == 2) asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(f) : "v"(v));
    else asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(f) : "v"(v));
    return f;
}

// RoPE (rotate-half, rope_heads ops.rs:693-740): element d of one rotated
// head whose pair-permuted projection is `src` (pair i at src[2i],
// src[2i+1]): x1' = x1*cos - x2*sin, x2' = x2*cos + x1*sin, each product and
// the sum rounded separately, with cos/sin rows cr/sr of the position.
__device__ __forceinline__ float rope_elem(const float *src, int d, int half, int rotary_dim, const float *cr,
                                           const float *sr) {
    if (d >= rotary_dim) return src[d];
    const int i = d < half ? d : d - half;
    const float a = src[2 * i], b = src[2 * i + 1], c = cr[i], s = sr[i];
    return d < half ? a * c - b * s : b * c + a * s;
}

// Cross-lane reductions with DPP row permutations (register-to-register,
// no LDS round trip) inside each row of 16 lanes, then the four row results
// read into a scalar. Steps, each exact once the previous one made its
// sub-groups uniform: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1]
// (lane ^ 2), row_half_mirror (lane 7 - i of 8: the other quad), row_mirror
// (lane 15 - i of 16: the other half row). The result is the same in every
// lane, with a fixed summation order.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over aligned groups of `W` consecutive lanes (W a power of two <= 16).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 16 && (W & (W - 1)) == 0, "group of 1..16 lanes");
    if constexpr (W >= 2) v += dpp_mov<kDppXor1>(v);
    if constexpr (W >= 4) v += dpp_mov<kDppXor2>(v);
    if constexpr (W >= 8) v += dpp_mov<kDppHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_mov<kDppMirror>(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppMirror>(v));
    return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

}  // namespace chip
