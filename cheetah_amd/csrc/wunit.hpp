// In-register decoding of the reference weight layouts, shared by the GEMV
// kernels and the persistent decode kernel.
//
// A "unit" is UB bytes of one row (16 = dwordx4 when every row start is
// 16-byte aligned, 4 = dword otherwise, as Q4's 4-byte row padding needs),
// holding E consecutive elements:
//   BF16: 2 per dword, value = bits << 16 (exact);
//   Q8:   4 int8 codes per dword (q8.rs:1-25);
//   Q4:   8 int4 codes per dword, nibble n of a dword is column 8*word + n,
//         low nibble = even column (q4.rs:12-24), sign-extended.
// Q8/Q4 return the integer code; the row scale multiplies the row sum.
#pragma once

#include "common.hpp"

namespace chip {

template <int FMT, int UB>
struct Unit;

template <int UB>
struct Unit<FMT_BF16, UB> {
    static constexpr int E = UB / 2;
    static constexpr int D = UB / 4;
    template <class F>
    __device__ static void decode(const uint32_t (&raw)[D], F &&f) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            f(2 * d, bf16_lo(raw[d]));
            f(2 * d + 1, bf16_hi(raw[d]));
        }
    }
    __device__ static float element(const uint8_t *row, int e) { return bf16_f32(*(const uint16_t *)(row + 2 * e)); }
};

template <int UB>
struct Unit<FMT_Q8, UB> {
    static constexpr int E = UB;
    static constexpr int D = UB / 4;
    template <class F>
    __device__ static void decode(const uint32_t (&raw)[D], F &&f) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
            for (int b = 0; b < 4; ++b) f(4 * d + b, (float)(int)(int8_t)(raw[d] >> (8 * b)));
        }
    }
    __device__ static float element(const uint8_t *row, int e) { return (float)(int8_t)row[e]; }
};

template <int UB>
struct Unit<FMT_Q4, UB> {
    static constexpr int E = UB * 2;
    static constexpr int D = UB / 4;
    template <class F>
    __device__ static void decode(const uint32_t (&raw)[D], F &&f) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
            for (int n = 0; n < 8; ++n) f(8 * d + n, (float)(((int)(raw[d] << (28 - 4 * n))) >> 28));
        }
    }
    __device__ static float element(const uint8_t *row, int e) {
        const uint8_t byte = row[e >> 1];
        const int nib = (e & 1) ? (byte >> 4) : (byte & 0xF);
        return (float)(nib >= 8 ? nib - 16 : nib);
    }
};

template <int UB>
__device__ __forceinline__ void load_raw(const uint8_t *p, uint32_t (&raw)[UB / 4]) {
    if constexpr (UB == 16) {
        const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
        raw[0] = v[0];
        raw[1] = v[1];
        raw[2] = v[2];
        raw[3] = v[3];
    } else {
        raw[0] = __builtin_nontemporal_load((const uint32_t *)p);
    }
}

}  // namespace chip
