// Decode GEMV y = W x for BF16 / Q8 / Q4 weights in the reference layouts
// (ops.rs:246 gemv, 544 gemv_q8, 586 gemv_q4). HBM-bound: each weight byte is
// read once, dequantized in registers (BF16: bits << 16; Q8/Q4: sign-extended
// code, row scale applied once to the row sum) and FMA'd against x held in LDS.
//
// Work split: a group of KS waves owns R consecutive rows; its 64*KS lanes
// stride along K in "units" of UB bytes (16 = dwordx4 when every row start
// is 16-byte aligned, else 4 = dword, which Q4's 4-byte row padding needs)
// and the KS partial sums meet in LDS in a fixed order. Blocks are 4 waves
// and stride over row groups, so a fused RMSNorm prologue runs once per
// block. The first weight loads are issued before the prologue and the
// stream is double-buffered in registers, so weight traffic starts at once
// and overlaps the x staging.
#include "kernels.hpp"
#include "wunit.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct Args {
    const uint8_t *w, *w2;
    const float *sc, *sc2;
    size_t stride;
    int rows, K;
    const float *x;
    const uint16_t *gain;
    float eps;
    const float *bias;
    float *y;
    float *residual;
    int epi;
};

template <int FMT, int UB, int R, int KS, bool NORM, bool DUAL>
__global__ __launch_bounds__(kThreads) void gemv_kernel(Args a) {
    using U = Unit<FMT, UB>;
    constexpr int E = U::E;
    constexpr int D = U::D;
    constexpr int UNROLL = UB == 16 ? 2 : 4;
    constexpr int GPB = kWaves / KS;        // row groups per block
    constexpr int STEP = 64 * KS * UNROLL;  // units per batch of one group
    constexpr int NM = DUAL ? 2 : 1;        // matrices read
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    __shared__ float kred[kWaves][NM * R];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int sub = wave % KS, gib = wave / KS;
    const int klane = sub * 64 + lane;
    const int K = a.K;
    const int n_units = K / E;
    const int groups = (a.rows + R - 1) / R;

    const uint8_t *rp[NM][R];
    auto set_rows = [&](int group) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(group * R + r, a.rows - 1);
            rp[0][r] = a.w + (size_t)row * a.stride;
            if constexpr (DUAL) rp[1][r] = a.w2 + (size_t)row * a.stride;
        }
    };
    uint32_t cur[UNROLL][NM][R][D];
    auto load_batch = [&](uint32_t (&buf)[UNROLL][NM][R][D], int u0) {
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) {
            const int u = u0 + 64 * KS * i;
            if (u < n_units) {
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) load_raw<UB>(rp[m][r] + (size_t)u * UB, buf[i][m][r]);
            }
        }
    };

    // Start this block's first weight loads, then stage x while they fly.
    int base = blockIdx.x * GPB;
    if (base + gib < groups) {
        set_rows(base + gib);
        load_batch(cur, klane);
    }
    if constexpr (NORM) {
        // RMSNorm (ops.rs:646-652): x * (inv * gain), inv = 1/sqrt(mean(x^2)+eps).
        float ss = 0.f;
        for (int i = tid; i < K; i += kThreads) {
            const float v = a.x[i];
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total += red[w];
        const float inv = 1.0f / sqrtf(total / (float)K + a.eps);
        for (int i = tid; i < K; i += kThreads) xs[i] = a.x[i] * (inv * bf16_f32(a.gain[i]));
    } else {
        for (int i = tid; i < K; i += kThreads) xs[i] = a.x[i];
    }
    __syncthreads();

    for (; base < groups; base += gridDim.x * GPB) {
        const int group = base + gib;
        const bool valid = group < groups;
        float acc[NM][R];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
        if (valid) {
            for (int u0 = klane; u0 < n_units; u0 += STEP) {
                uint32_t nxt[UNROLL][NM][R][D];
                const bool more = u0 + STEP < n_units;
                if (more) load_batch(nxt, u0 + STEP);
#pragma unroll
                for (int i = 0; i < UNROLL; ++i) {
                    const int u = u0 + 64 * KS * i;
                    if (u < n_units) {
                        const float *xu = xs + u * E;
#pragma unroll
                        for (int m = 0; m < NM; ++m)
#pragma unroll
                            for (int r = 0; r < R; ++r)
                                U::decode(cur[i][m][r], [&](int e, float wv) { acc[m][r] = fmaf(wv, xu[e], acc[m][r]); });
                    }
                }
                if (more) {
#pragma unroll
                    for (int i = 0; i < UNROLL; ++i)
#pragma unroll
                        for (int m = 0; m < NM; ++m)
#pragma unroll
                            for (int r = 0; r < R; ++r)
#pragma unroll
                                for (int d = 0; d < D; ++d) cur[i][m][r][d] = nxt[i][m][r][d];
                }
            }
            // Ragged tail (K not a multiple of the unit width).
            for (int e = n_units * E + klane; e < K; e += 64 * KS) {
                const float xv = xs[e];
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[m][r] = fmaf(U::element(rp[m][r], e), xv, acc[m][r]);
            }
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);
        // Prefetch the next group's first batch before the epilogue.
        const int nbase = base + gridDim.x * GPB;
        if (nbase + gib < groups) {
            set_rows(nbase + gib);
            load_batch(cur, klane);
        }
        if constexpr (KS > 1) {
            if (lane == 0) {
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) kred[wave][m * R + r] = acc[m][r];
            }
            __syncthreads();
            if (sub == 0) {
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float s = kred[wave][m * R + r];
#pragma unroll
                        for (int k = 1; k < KS; ++k) s += kred[wave + k][m * R + r];
                        acc[m][r] = s;
                    }
            }
            __syncthreads();
        }
        if (sub == 0 && valid) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = group * R + r;
                if (lane == r && row < a.rows) {
                    float v = acc[0][r];
                    if (a.sc) v = v * a.sc[row];
                    if constexpr (DUAL) {
                        float u = acc[1][r];
                        if (a.sc2) u = u * a.sc2[row];
                        // silu_multiply, ops.rs:743-747: g * (u / (1 + exp(-g))).
                        a.y[row] = v * (u / (1.0f + expf(-v)));
                    } else {
                        if (a.bias) v = v + a.bias[row];
                        if (a.epi == EPI_RESIDUAL) a.residual[row] = a.residual[row] + v;
                        else a.y[row] = v;
                    }
                }
            }
        }
    }
}

template <int FMT, int UB, int R, int KS, bool NORM, bool DUAL>
int launch_t(const Args &a, hipStream_t s) {
    constexpr int GPB = kWaves / KS;
    const int groups = (a.rows + R - 1) / R;
    int blocks = (groups + GPB - 1) / GPB;
    if (NORM) blocks = min(blocks, 2048);
    const size_t lds = (size_t)a.K * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<FMT, UB, R, KS, NORM, DUAL>), dim3(blocks), dim3(kThreads), lds, s, a);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

// Rows per group and waves per group: enough waves to keep every CU busy
// (~8 per CU) while each lane still streams at least two units.
template <int FMT, int UB, bool NORM, bool DUAL>
int pick_shape(const Args &a, hipStream_t s) {
    constexpr int E = Unit<FMT, UB>::E;
    const int n_units = a.K / E;
    if (a.rows >= 16384) return launch_t<FMT, UB, 2, 1, NORM, DUAL>(a, s);
    int ks = 1;
    while (ks < 4 && a.rows * ks < 2048 && n_units >= 64 * ks * 2 * 2) ks *= 2;
    if (ks == 4) return launch_t<FMT, UB, 1, 4, NORM, DUAL>(a, s);
    if (ks == 2) return launch_t<FMT, UB, 1, 2, NORM, DUAL>(a, s);
    return launch_t<FMT, UB, 1, 1, NORM, DUAL>(a, s);
}

template <int FMT, bool NORM, bool DUAL>
int pick_ub(const Args &a, bool aligned16, hipStream_t s) {
    if (aligned16) return pick_shape<FMT, 16, NORM, DUAL>(a, s);
    return pick_shape<FMT, 4, NORM, DUAL>(a, s);
}

template <int FMT>
int pick_mode(const Args &a, bool aligned16, bool norm, bool dual, hipStream_t s) {
    if (norm) return dual ? pick_ub<FMT, true, true>(a, aligned16, s) : pick_ub<FMT, true, false>(a, aligned16, s);
    return dual ? pick_ub<FMT, false, true>(a, aligned16, s) : pick_ub<FMT, false, false>(a, aligned16, s);
}

}  // namespace

int launch_gemv(const GemvJob &job, hipStream_t s) {
    const WMat &w = job.w;
    if (!w.base || !job.x || w.rows == 0 || w.cols == 0) return fail("HIP backend: gemv needs a weight and an input.");
    if (w.rows > (size_t)INT32_MAX || w.cols > (size_t)INT32_MAX) return fail("HIP backend: gemv shape too large.");
    const bool dual = job.epi == EPI_SWIGLU;
    if (dual && (!job.w2.base || job.w2.fmt != w.fmt || job.w2.rows != w.rows || job.w2.cols != w.cols))
        return fail("HIP backend: SwiGLU gemv needs gate and up matrices of one shape and format.");
    if (job.epi == EPI_RESIDUAL ? !job.residual : !job.y) return fail("HIP backend: gemv has no output.");
    if ((size_t)w.cols * sizeof(float) + 256 > device_max_lds())
        return fail("HIP backend: gemv input width " + std::to_string(w.cols) + " exceeds the LDS staging limit.");
    Args a{};
    a.w = w.payload();
    a.sc = w.scales();
    a.w2 = dual ? job.w2.payload() : nullptr;
    a.sc2 = dual ? job.w2.scales() : nullptr;
    a.stride = w.row_stride();
    a.rows = (int)w.rows;
    a.K = (int)w.cols;
    a.x = job.x;
    a.gain = job.norm_gain;
    a.eps = job.eps;
    a.bias = job.bias;
    a.y = job.y;
    a.residual = job.residual;
    a.epi = job.epi;
    const bool aligned16 =
        a.stride % 16 == 0 && ((uintptr_t)a.w % 16) == 0 && (!dual || ((uintptr_t)a.w2 % 16) == 0);
    const bool norm = job.norm_gain != nullptr;
    switch (w.fmt) {
        case FMT_BF16: return pick_mode<FMT_BF16>(a, aligned16, norm, dual, s);
        case FMT_Q8: return pick_mode<FMT_Q8>(a, aligned16, norm, dual, s);
        case FMT_Q4: return pick_mode<FMT_Q4>(a, aligned16, norm, dual, s);
    }
    return fail("HIP backend: unknown weight format.");
}

}  // namespace chip
