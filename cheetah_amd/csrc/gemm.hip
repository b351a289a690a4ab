// Prefill GEMM Y[n, rows] = X[n, cols] · Wᵀ on the gfx950 matrix cores
// (the batched projections of forward_layer_chunk, qwen2.rs:240-426; gemm,
// ops.rs:308, and the per-row quantized linear_batch loop, ops.rs:1244-1326).
//
// Operands: W stays in the reference layout and is converted to BF16 while
// it is staged into LDS — BF16 as stored, Q8/Q4 codes exactly (|code| <= 127
// fits BF16's 8-bit significand) with the row scale applied to the f32 sum in
// the epilogue. X is f32; it is split into hi = bf16(x) and lo = bf16(x - hi)
// so two v_mfma_f32_32x32x16_bf16 per k-step carry x to ~2^-17 relative
// error (f32 accumulation), instead of bf16's 2^-9.
//
// Tiling: a 256-thread block computes a 64 (tokens) x 64 (weight rows) tile
// as 2 x 2 waves of 32 x 32; K advances 64 per LDS stage.
#include "kernels.hpp"

namespace chip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BM = 64, BN = 64, BK = 64;
constexpr int LDK = BK + 8;  // LDS row stride in bf16 (pad breaks bank conflicts)

struct GArgs {
    const uint8_t *w, *w2;
    const float *sc, *sc2;
    size_t stride;
    int N, K, M;  // N = weight rows, K = cols, M = tokens
    const float *x;
    const float *bias;
    float *y, *residual;
    int epi;
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// BF16 bits of a small integer code (exact).
__device__ __forceinline__ uint16_t code_bf16(int code) { return (uint16_t)(__float_as_uint((float)code) >> 16); }

// Stage a BN x BK tile of W (rows n0.., k0..) into LDS as BF16 bits.
template <int FMT>
__device__ __forceinline__ void stage_w(const GArgs &a, const uint8_t *w, int n0, int k0, uint16_t *ws) {
    const int tid = threadIdx.x;
    if constexpr (FMT == FMT_BF16) {
        // 64 rows x 64 k = 64 x 128 B: 512 chunks of 16 B (8 k), 2 per thread.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kThreads;
            const int r = c >> 3, kc = (c & 7) * 8;
            const int n = n0 + r, k = k0 + kc;
            uint32_t v[4] = {0, 0, 0, 0};
            if (n < a.N) {
                const uint16_t *src = (const uint16_t *)(w + (size_t)n * a.stride) + k;
                if (k + 8 <= a.K && (a.stride % 16) == 0) {
                    u32x4 t = *(const u32x4 *)src;
                    v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = (k + q < a.K) ? src[q] : 0;
                    v[0] = pack2(e[0], e[1]); v[1] = pack2(e[2], e[3]);
                    v[2] = pack2(e[4], e[5]); v[3] = pack2(e[6], e[7]);
                }
            }
            *(u32x4 *)(ws + r * LDK + kc) = u32x4{v[0], v[1], v[2], v[3]};
        }
    } else if constexpr (FMT == FMT_Q8) {
        // 64 rows x 64 codes: 256 chunks of 16 codes, 1 per thread.
        const int r = tid >> 2, kc = (tid & 3) * 16;
        const int n = n0 + r, k = k0 + kc;
        uint16_t e[16];
        if (n < a.N) {
            const int8_t *src = (const int8_t *)(w + (size_t)n * a.stride) + k;
            if (k + 16 <= a.K && (a.stride % 16) == 0 && ((uintptr_t)src % 16) == 0) {
                u32x4 t = *(const u32x4 *)src;
#pragma unroll
                for (int q = 0; q < 16; ++q) e[q] = code_bf16((int)(int8_t)(t[q >> 2] >> (8 * (q & 3))));
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) e[q] = (k + q < a.K) ? code_bf16(src[q]) : 0;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) e[q] = 0;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            *(u32x4 *)(ws + r * LDK + kc + 8 * h) =
                u32x4{pack2(e[8 * h], e[8 * h + 1]), pack2(e[8 * h + 2], e[8 * h + 3]),
                      pack2(e[8 * h + 4], e[8 * h + 5]), pack2(e[8 * h + 6], e[8 * h + 7])};
    } else {
        // Q4: 64 rows x 64 codes = 64 x 32 B; rows are only 4-byte aligned.
        const int r = tid >> 2, kc = (tid & 3) * 16;
        const int n = n0 + r, k = k0 + kc;
        uint16_t e[16];
        if (n < a.N) {
            const uint8_t *src = w + (size_t)n * a.stride + (k >> 1);
            if (k + 16 <= a.K) {
                const uint32_t d0 = *(const uint32_t *)src, d1 = *(const uint32_t *)(src + 4);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    e[q] = code_bf16(((int)(d0 << (28 - 4 * q))) >> 28);
                    e[8 + q] = code_bf16(((int)(d1 << (28 - 4 * q))) >> 28);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    int code = 0;
                    if (k + q < a.K) {
                        const uint8_t byte = src[q >> 1];
                        const int nib = (q & 1) ? (byte >> 4) : (byte & 0xF);
                        code = nib >= 8 ? nib - 16 : nib;
                    }
                    e[q] = code_bf16(code);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) e[q] = 0;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            *(u32x4 *)(ws + r * LDK + kc + 8 * h) =
                u32x4{pack2(e[8 * h], e[8 * h + 1]), pack2(e[8 * h + 2], e[8 * h + 3]),
                      pack2(e[8 * h + 4], e[8 * h + 5]), pack2(e[8 * h + 6], e[8 * h + 7])};
    }
}

// Stage a BM x BK tile of X (f32) into LDS as hi / lo BF16 halves.
__device__ __forceinline__ void stage_x(const GArgs &a, int m0, int k0, uint16_t *xh, uint16_t *xl) {
    const int tid = threadIdx.x;
    // 64 rows x 64 k f32 = 1024 chunks of 4 floats, 4 per thread.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + i * kThreads;
        const int r = c >> 4, kc = (c & 15) * 4;
        const int m = m0 + r, k = k0 + kc;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (m < a.M) {
            const float *src = a.x + (size_t)m * a.K + k;
            if (k + 4 <= a.K && (a.K % 4) == 0) {
                f32x4 t = *(const f32x4 *)src;
                v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = (k + q < a.K) ? src[q] : 0.f;
            }
        }
        uint16_t h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h[q] = f32_bf16_rne(v[q]);
            l[q] = f32_bf16_rne(v[q] - bf16_f32(h[q]));
        }
        *(uint2 *)(xh + r * LDK + kc) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
        *(uint2 *)(xl + r * LDK + kc) = make_uint2(pack2(l[0], l[1]), pack2(l[2], l[3]));
    }
}

__device__ __forceinline__ bf16x8 frag(const uint16_t *base, int row, int k) {
    u32x4 t = *(const u32x4 *)(base + row * LDK + k);
    return __builtin_bit_cast(bf16x8, t);
}

template <int FMT, bool DUAL>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t xh[BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t xl[BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t ws[BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t ws2[DUAL ? BN * LDK : 8];

    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    f32x16 acc = {}, acc2 = {};

    for (int k0 = 0; k0 < a.K; k0 += BK) {
        stage_x(a, m0, k0, xh, xl);
        stage_w<FMT>(a, a.w, n0, k0, ws);
        if constexpr (DUAL) stage_w<FMT>(a, a.w2, n0, k0, ws2);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            const int kf = kk + 8 * (lane >> 5);
            const bf16x8 ah = frag(xh, wm + (lane & 31), kf);
            const bf16x8 al = frag(xl, wm + (lane & 31), kf);
            const bf16x8 b = frag(ws, wn + (lane & 31), kf);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b, acc, 0, 0, 0);
            if constexpr (DUAL) {
                const bf16x8 b2 = frag(ws2, wn + (lane & 31), kf);
                acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b2, acc2, 0, 0, 0);
                acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b2, acc2, 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // D layout of the 32x32 MFMA: column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4.
    const int n = n0 + wn + (lane & 31);
    if (n >= a.N) return;
    const float sc = a.sc ? a.sc[n] : 1.0f;
    const float sc2 = (DUAL && a.sc2) ? a.sc2[n] : 1.0f;
    const float b = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= a.M) continue;
        float v = a.sc ? acc[r] * sc : acc[r];
        const size_t o = (size_t)m * a.N + n;
        if constexpr (DUAL) {
            const float u = a.sc2 ? acc2[r] * sc2 : acc2[r];
            a.y[o] = v * (u / (1.0f + expf(-v)));
        } else {
            if (a.bias) v = v + b;
            if (a.epi == EPI_RESIDUAL) a.residual[o] = a.residual[o] + v;
            else a.y[o] = v;
        }
    }
}

template <int FMT>
int launch_fmt(const GArgs &a, bool dual, hipStream_t s) {
    dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
    if (dual) hipLaunchKernelGGL((gemm_kernel<FMT, true>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((gemm_kernel<FMT, false>), grid, dim3(kThreads), 0, s, a);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

}  // namespace

int launch_gemm(const GemmJob &job, hipStream_t s) {
    const WMat &w = job.w;
    if (job.n == 0) return 0;
    if (!w.base || !job.x || w.rows == 0 || w.cols == 0) return fail("HIP backend: gemm needs a weight and an input.");
    if (w.rows > (size_t)INT32_MAX || w.cols > (size_t)INT32_MAX || job.n > 65535u * BM)
        return fail("HIP backend: gemm shape too large.");
    const bool dual = job.epi == EPI_SWIGLU;
    if (dual && (!job.w2.base || job.w2.fmt != w.fmt || job.w2.rows != w.rows || job.w2.cols != w.cols))
        return fail("HIP backend: SwiGLU gemm needs gate and up matrices of one shape and format.");
    if (job.epi == EPI_RESIDUAL ? !job.residual : !job.y) return fail("HIP backend: gemm has no output.");
    GArgs a{};
    a.w = w.payload();
    a.sc = w.scales();
    a.w2 = dual ? job.w2.payload() : nullptr;
    a.sc2 = dual ? job.w2.scales() : nullptr;
    a.stride = w.row_stride();
    a.N = (int)w.rows;
    a.K = (int)w.cols;
    a.M = (int)job.n;
    a.x = job.x;
    a.bias = job.bias;
    a.y = job.y;
    a.residual = job.residual;
    a.epi = job.epi;
    switch (w.fmt) {
        case FMT_BF16: return launch_fmt<FMT_BF16>(a, dual, s);
        case FMT_Q8: return launch_fmt<FMT_Q8>(a, dual, s);
        case FMT_Q4: return launch_fmt<FMT_Q4>(a, dual, s);
    }
    return fail("HIP backend: unknown weight format.");
}

}  // namespace chip
