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
// Tiling: a block of 4 or 8 waves (2 x 2 or 4 x 2) computes 64 or 128
// tokens x 128 weight rows, each wave 32 tokens x 64 rows (the register-
// staged fallback also 64 x 64 per wave); K advances 32 per LDS stage, the
// next stages' copies in flight during the MFMAs.
//
// Accumulation order: K is cut into chunks of a depth fixed by K alone; each
// chunk is accumulated from zero. A single matrix's n chunk sums are folded
// as two halves, t = (c0 + ... + c(h-1)) + (ch + ... + c(n-1)) with
// h = ceil(n / 2), each half left to right (for n <= 3 this is the plain left
// fold); the dual gate/up GEMM folds its chunks left to right. With many tiles
// a block folds its chunks in registers; with fewer tiles the chunks go to
// split-K blocks (every chunk its own block, or a single matrix's two halves
// one block each) and the stored sums are folded by a reduce kernel or by the
// kernel that reads the output, in the same association. Every path gives
// the same bits, so a token's outputs never depend on how many tokens share
// the call (chunked prefill stays bit-exact however the prompt is cut).
#include <algorithm>
#include <cstdlib>

#include "kernels.hpp"

namespace chip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BN = 128, BK = 32;
constexpr int LDK = BK + 8;  // 80-byte LDS rows: 16 consecutive rows start on distinct bank groups

struct GArgs {
    const uint8_t *w, *w2;
    const float *sc, *sc2;
    size_t stride;
    int N, K, M;  // N = weight rows, K = cols, M = tokens
    const float *x;
    const uint16_t *xh, *xl;  // x pre-split into hi / lo BF16 halves, [M][K] (or null)
    const float *bias;
    float *y, *residual;
    uint16_t *yh, *yl;  // SwiGLU: the output also as BF16 halves (or null)
    int defer;          // split-K: leave the chunk sums for the caller
    int epi;
    int chunk, nchunks;  // accumulation chunk depth (multiple of BK) and count
    int nstored;         // split-K: sums stored per output (nchunks, or 2 halves of a single matrix)
    float *ws;           // split-K: [nstored][M][N] sums (a second set for the dual matrix)
    int vec_x, vec_w;    // 16-byte global loads allowed
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// BF16 bits of a small integer code (exact).
__device__ __forceinline__ uint16_t code_bf16(int code) { return (uint16_t)(__float_as_uint((float)code) >> 16); }

__device__ __forceinline__ bf16x8 frag(const uint16_t *base, int row, int k) {
    return __builtin_bit_cast(bf16x8, *(const u32x4 *)(base + row * LDK + k));
}

// One stage's operands in flight: X as f32, W as raw reference bytes.
template <int MT>
struct Regs {
    static constexpr int XV = 64 * MT * BK / 4 / kThreads;  // float4 per thread
    static constexpr int XB = 64 * MT * BK / 8 / kThreads;  // 8-element BF16 chunks per thread
    f32x4 x[XV];
    u32x4 xh[XB], xl[XB];
    u32x4 w[2];   // BF16: 2 x 8 elements; Q8: w[0] = 16 codes; Q4: w[0].xy = 16 codes
    u32x4 w2[2];  // dual matrix
};

template <int MT>
__device__ __forceinline__ void load_x(const GArgs &a, int m0, int k0, Regs<MT> &r) {
#pragma unroll
    for (int i = 0; i < Regs<MT>::XV; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int row = c >> 3, kc = (c & 7) * 4;
        const int m = m0 + row, k = k0 + kc;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (m < a.M && k < a.K) {
            const float *src = a.x + (size_t)m * a.K + k;
            if (a.vec_x) {
                v = *(const f32x4 *)src;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = k + q < a.K ? src[q] : 0.f;
            }
        }
        r.x[i] = v;
    }
}

// Pre-split x: BM x BK BF16 per half, 16-byte chunks (K % 8 == 0).
template <int MT>
__device__ __forceinline__ void load_xs(const GArgs &a, int m0, int k0, Regs<MT> &r) {
#pragma unroll
    for (int i = 0; i < Regs<MT>::XB; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int row = c >> 2, kc = (c & 3) * 8;
        const int m = m0 + row, k = k0 + kc;
        if (m < a.M && k < a.K) {
            r.xh[i] = *(const u32x4 *)(a.xh + (size_t)m * a.K + k);
            r.xl[i] = *(const u32x4 *)(a.xl + (size_t)m * a.K + k);
        } else {
            r.xh[i] = u32x4{0u, 0u, 0u, 0u};
            r.xl[i] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

template <int MT>
__device__ __forceinline__ void store_xs(const Regs<MT> &r, uint16_t *xh, uint16_t *xl) {
#pragma unroll
    for (int i = 0; i < Regs<MT>::XB; ++i) {
        const int c = threadIdx.x + kThreads * i;
        *(u32x4 *)(xh + (c >> 2) * LDK + (c & 3) * 8) = r.xh[i];
        *(u32x4 *)(xl + (c >> 2) * LDK + (c & 3) * 8) = r.xl[i];
    }
}

template <int MT>
__device__ __forceinline__ void store_x(const Regs<MT> &r, uint16_t *xh, uint16_t *xl) {
#pragma unroll
    for (int i = 0; i < Regs<MT>::XV; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int row = c >> 3, kc = (c & 7) * 4;
        uint16_t h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const __bf16 hb = (__bf16)r.x[i][q];
            h[q] = __builtin_bit_cast(uint16_t, hb);
            l[q] = __builtin_bit_cast(uint16_t, (__bf16)(r.x[i][q] - (float)hb));
        }
        *(uint2 *)(xh + row * LDK + kc) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
        *(uint2 *)(xl + row * LDK + kc) = make_uint2(pack2(l[0], l[1]), pack2(l[2], l[3]));
    }
}

// W stage: BN rows x BK columns of the reference layout.
template <int FMT>
__device__ __forceinline__ void load_w(const GArgs &a, const uint8_t *w, int n0, int k0, u32x4 (&out)[2]) {
    const int tid = threadIdx.x;
    if constexpr (FMT == FMT_BF16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = tid + kThreads * j;
            const int row = c >> 2, kc = (c & 3) * 8;
            const int n = n0 + row, k = k0 + kc;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (n < a.N && k < a.K) {
                const uint16_t *src = (const uint16_t *)(w + (size_t)n * a.stride) + k;
                if (a.vec_w) {
                    v = *(const u32x4 *)src;
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = k + q < a.K ? src[q] : 0;
                    v = u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7])};
                }
            }
            out[j] = v;
        }
    } else {
        // Q8 / Q4: 16 codes per thread, rows tid / 2, codes 16 (tid % 2) ..
        const int row = tid >> 1, kc = (tid & 1) * 16;
        const int n = n0 + row, k = k0 + kc;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (n < a.N && k < a.K) {
            const uint8_t *rp = w + (size_t)n * a.stride;
            if constexpr (FMT == FMT_Q8) {
                if (a.vec_w) {
                    v = *(const u32x4 *)(rp + k);
                } else {
                    uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        if (k + q < a.K) d[q >> 2] |= (uint32_t)rp[k + q] << (8 * (q & 3));
                    v = u32x4{d[0], d[1], d[2], d[3]};
                }
            } else {
                // Rows are 4-byte aligned; k is a multiple of 16, so the 8 code
                // bytes are 8-byte aligned within the row.
                if (k + 16 <= a.K) {
                    const uint32_t *p = (const uint32_t *)(rp + (k >> 1));
                    v = u32x4{p[0], p[1], 0u, 0u};
                } else {
                    uint32_t d[2] = {0u, 0u};
                    for (int q = 0; q < 16 && k + q < a.K; ++q) {
                        const uint8_t byte = rp[(k + q) >> 1];
                        const uint32_t nib = ((k + q) & 1) ? (byte >> 4) : (byte & 0xF);
                        d[q >> 3] |= nib << (4 * (q & 7));
                    }
                    v = u32x4{d[0], d[1], 0u, 0u};
                }
            }
        }
        out[0] = v;
    }
}

template <int FMT>
__device__ __forceinline__ void store_w(const u32x4 (&in)[2], uint16_t *ws) {
    const int tid = threadIdx.x;
    if constexpr (FMT == FMT_BF16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = tid + kThreads * j;
            *(u32x4 *)(ws + (c >> 2) * LDK + (c & 3) * 8) = in[j];
        }
    } else {
        const int row = tid >> 1, kc = (tid & 1) * 16;
        uint16_t e[16];
        if constexpr (FMT == FMT_Q8) {
#pragma unroll
            for (int q = 0; q < 16; ++q) e[q] = code_bf16((int)(int8_t)(in[0][q >> 2] >> (8 * (q & 3))));
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) e[q] = code_bf16(((int)(in[0][q >> 3] << (28 - 4 * (q & 7)))) >> 28);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            *(u32x4 *)(ws + row * LDK + kc + 8 * h) =
                u32x4{pack2(e[8 * h], e[8 * h + 1]), pack2(e[8 * h + 2], e[8 * h + 3]),
                      pack2(e[8 * h + 4], e[8 * h + 5]), pack2(e[8 * h + 6], e[8 * h + 7])};
    }
}

// out = f(v * row scale (+ bias)); dual: SwiGLU of gate v and up u.
template <bool DUAL>
__device__ __forceinline__ void epilogue(const GArgs &a, int m, int n, float v, float u) {
    if (a.sc) v = v * a.sc[n];
    const size_t o = (size_t)m * a.N + n;
    if constexpr (DUAL) {
        if (a.sc2) u = u * a.sc2[n];
        // silu_multiply, ops.rs:743-747: g * (u / (1 + exp(-g))).
        const float g = v * (u / (1.0f + expf(-v)));
        a.y[o] = g;
        if (a.yh) {
            const __bf16 hb = (__bf16)g;
            a.yh[o] = __builtin_bit_cast(uint16_t, hb);
            a.yl[o] = __builtin_bit_cast(uint16_t, (__bf16)(g - (float)hb));
        }
    } else {
        if (a.bias) v = v + a.bias[n];
        if (a.epi == EPI_RESIDUAL) a.residual[o] = a.residual[o] + v;
        else a.y[o] = v;
    }
}

// The epilogue for one lane's outputs of a finished tile: column n per j,
// rows m = mbase + 32 i + 8 (q / 4) + 4 (lane / 32) + q % 4. The column's scale
// and bias, then a 32-row block's residuals, are loaded before any store (one
// wait instead of one per output); each output's arithmetic is epilogue's.
template <bool DUAL, int MT>
__device__ __forceinline__ void epilogue_tile(const GArgs &a, const f32x16 (&tot)[MT][2],
                                              const f32x16 (&tot2)[DUAL ? MT : 1][2], int mbase, int nbase, int lane) {
    const bool resid = !DUAL && a.epi == EPI_RESIDUAL;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = nbase + 32 * j + (lane & 31);
        if (n >= a.N) continue;
        const float scn = a.sc ? a.sc[n] : 1.0f;
        const float sc2n = DUAL && a.sc2 ? a.sc2[n] : 1.0f;
        const float bn = !DUAL && a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            float res[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = mbase + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                res[q] = resid && m < a.M ? a.residual[(size_t)m * a.N + n] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = mbase + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                if (m >= a.M) continue;
                const size_t o = (size_t)m * a.N + n;
                float v = tot[i][j][q];
                if (a.sc) v = v * scn;
                if constexpr (DUAL) {
                    float u = tot2[i][j][q];
                    if (a.sc2) u = u * sc2n;
                    // silu_multiply, ops.rs:743-747: g * (u / (1 + exp(-g))).
                    const float g = v * (u / (1.0f + expf(-v)));
                    a.y[o] = g;
                    if (a.yh) {
                        const __bf16 hb = (__bf16)g;
                        a.yh[o] = __builtin_bit_cast(uint16_t, hb);
                        a.yl[o] = __builtin_bit_cast(uint16_t, (__bf16)(g - (float)hb));
                    }
                } else {
                    if (a.bias) v = v + bn;
                    if (resid) a.residual[o] = res[q] + v;
                    else a.y[o] = v;
                }
            }
        }
    }
}

// Output tile of this block. Blocks are numbered so that the token tiles of
// one weight-row tile are consecutive, and (with the 8 XCDs taking block ids
// round-robin) run on one XCD: each weight tile streams from HBM about once
// and the block's neighbours find it in that XCD's L2, instead of every token
// tile re-reading the whole matrix.
__device__ __forceinline__ void tile_of(int nN, int nM, int &n0, int &m0, int BMt) {
    const int total = nN * nM, bid = blockIdx.x;
    const int lid = total % 8 == 0 ? (bid % 8) * (total / 8) + bid / 8 : bid;
    m0 = (lid % nM) * BMt;
    n0 = (lid / nM) * BN;
}

// blockIdx: x = output tile (tile_of), z = chunk (split-K) or 0.
template <int FMT, bool DUAL, int MT, bool PRE>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GArgs a, int split) {
    constexpr int BM = 64 * MT;
    __shared__ __attribute__((aligned(16))) uint16_t xh[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t xl[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t wsm[2][BN * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t wsm2[DUAL ? 2 : 1][DUAL ? BN * LDK : 8];

    int n0, m0;
    tile_of((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, n0, m0, BM);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 32 * MT, wn = (wave & 1) * 64;
    const int kbeg = split ? blockIdx.z * a.chunk : 0;
    const int kend = split ? min(a.K, kbeg + a.chunk) : a.K;
    // Single matrix, folding in registers: the first half's total moves to
    // th when the second half begins (two-half association).
    const int khalf = (a.nchunks + 1) / 2 * a.chunk;

    f32x16 acc[MT][2], acc2[DUAL ? MT : 1][2], tot[MT][2], tot2[DUAL ? MT : 1][2], th[DUAL ? 1 : MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[i][j] = f32x16{};
            tot[i][j] = f32x16{};
            if constexpr (DUAL) {
                acc2[i][j] = f32x16{};
                tot2[i][j] = f32x16{};
            } else {
                th[i][j] = f32x16{};
            }
        }

    Regs<MT> r;
    if constexpr (PRE) load_xs<MT>(a, m0, kbeg, r);
    else load_x<MT>(a, m0, kbeg, r);
    load_w<FMT>(a, a.w, n0, kbeg, r.w);
    if constexpr (DUAL) load_w<FMT>(a, a.w2, n0, kbeg, r.w2);
    if constexpr (PRE) store_xs<MT>(r, xh[0], xl[0]);
    else store_x<MT>(r, xh[0], xl[0]);
    store_w<FMT>(r.w, wsm[0]);
    if constexpr (DUAL) store_w<FMT>(r.w2, wsm2[0]);
    __syncthreads();
    int b = 0;
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) {
            if constexpr (PRE) load_xs<MT>(a, m0, k0 + BK, r);
            else load_x<MT>(a, m0, k0 + BK, r);
            load_w<FMT>(a, a.w, n0, k0 + BK, r.w);
            if constexpr (DUAL) load_w<FMT>(a, a.w2, n0, k0 + BK, r.w2);
        }
#pragma unroll
        for (int ks = 0; ks < BK; ks += 16) {
            const int kf = ks + 8 * (lane >> 5);
            bf16x8 ah[MT], al[MT], bw[2], bw2[DUAL ? 2 : 1];
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                ah[i] = frag(xh[b], wm + 32 * i + (lane & 31), kf);
                al[i] = frag(xl[b], wm + 32 * i + (lane & 31), kf);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                bw[j] = frag(wsm[b], wn + 32 * j + (lane & 31), kf);
                if constexpr (DUAL) bw2[j] = frag(wsm2[b], wn + 32 * j + (lane & 31), kf);
            }
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bw[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bw[j], acc[i][j], 0, 0, 0);
                    if constexpr (DUAL) {
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bw2[j], acc2[i][j], 0, 0, 0);
                        acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bw2[j], acc2[i][j], 0, 0, 0);
                    }
                }
        }
        // Chunk end: fold the chunk sum into the running total (t += c); a
        // single matrix's first half ends here: th = t, t = 0.
        if (k0 + BK >= kend || ((k0 + BK) % a.chunk) == 0) {
            const bool half_end = !DUAL && !split && k0 + BK == khalf && khalf < kend;
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    tot[i][j] += acc[i][j];
                    acc[i][j] = f32x16{};
                    if constexpr (DUAL) {
                        tot2[i][j] += acc2[i][j];
                        acc2[i][j] = f32x16{};
                    } else if (half_end) {
                        th[i][j] = tot[i][j];
                        tot[i][j] = f32x16{};
                    }
                }
        }
        if (more) {
            if constexpr (PRE) store_xs<MT>(r, xh[b ^ 1], xl[b ^ 1]);
            else store_x<MT>(r, xh[b ^ 1], xl[b ^ 1]);
            store_w<FMT>(r.w, wsm[b ^ 1]);
            if constexpr (DUAL) store_w<FMT>(r.w2, wsm2[b ^ 1]);
        }
        __syncthreads();
        b ^= 1;
    }
    // D layout of the 32x32 MFMA: column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4.
    if (!split) {
        if constexpr (!DUAL) {
            if (khalf < kend) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) tot[i][j] = th[i][j] + tot[i][j];
            }
        }
        epilogue_tile<DUAL, MT>(a, tot, tot2, m0 + wm, n0 + wn, lane);
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        if (n >= a.N) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = m0 + wm + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                if (m >= a.M) continue;
                const size_t o = ((size_t)blockIdx.z * a.M + m) * a.N + n;
                a.ws[o] = tot[i][j][q];
                if constexpr (DUAL) a.ws[(size_t)a.nstored * a.M * a.N + o] = tot2[i][j][q];
            }
    }
}

// LDS tiles are unpadded 32-element (64-byte) rows; 16-byte chunk c of row r
// sits at slot c ^ ((r / 4) % 4), which keeps the fragment reads of 16
// consecutive rows on distinct LDS banks.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 2) & 3); }

template <bool DUAL>
__global__ __launch_bounds__(kThreads) void gemm_reduce_kernel(GArgs a);

// s_waitcnt immediate waiting until at most n vector-memory ops are pending.
constexpr int vm_wait_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// ---------------------------------------------------------------------------
// Ring GEMM, every weight format (x pre-split, K % 32 == 0). Per 32-wide K
// stage the block's x halves and its raw weight bytes (BF16 rows, Q8 codes,
// Q4 nibbles) go global -> LDS by buffer loads that write LDS directly: a
// lane's source offset is fixed for the whole launch and the stage's K
// offset is a scalar, so issuing a stage costs no vector instructions. The
// ring holds NS = 4 stages (6 measured no faster); stage s + NS - 2 is issued
// while stage s computes.
// Q8/Q4 codes of stage s + 1 are converted to BF16 (exactly) once per block,
// 16 (4 waves) or 8 (8 waves) per thread, into one of three converted tiles
// after stage s's MFMAs;
// BF16 weights are read straight from the ring. One barrier per stage. The
// MFMA sequence per output and the chunk folds are those of gemm_kernel, so
// the results are the same bits.
// ---------------------------------------------------------------------------
template <int FMT>
constexpr int ring_w_row_bytes() { return FMT == FMT_BF16 ? 64 : FMT == FMT_Q8 ? 32 : 16; }

// Tokens per block: WV waves as WV / 2 x 2, each 32 MT tokens x 64 rows.
template <int MT, int WV>
constexpr int ring_bm() { return 32 * MT * (WV / 2); }

template <int FMT, bool DUAL, int MT, int NS, int WV>
constexpr size_t ring_lds_bytes() {
    constexpr size_t slot = 2 * ring_bm<MT, WV>() * 64 + (DUAL ? 2 : 1) * BN * ring_w_row_bytes<FMT>();
    return NS * slot + (FMT == FMT_BF16 ? 0 : 3 * (DUAL ? 2 : 1) * BN * 64);
}

// Weight copy granule (bytes per lane) of the ring: Q4 rows are only 4-byte
// aligned; Q8 stages are copied 4 bytes a lane where 16 would leave some of
// 8 waves without a copy (every wave must issue the same count).
template <int FMT, int WV>
constexpr int ring_w_granule() { return FMT == FMT_Q4 ? 4 : (FMT == FMT_Q8 && WV == 8) ? 4 : 16; }

typedef __attribute__((address_space(3))) void lds_void;

// size bytes per lane from buffer r at voffset + soffset into LDS at
// lds + size * lane (lds wave-uniform).
template <int SIZE>  // 16 or 4
__device__ __forceinline__ void buf_to_lds(__amdgpu_buffer_rsrc_t r, void *lds, int voffset, int soffset) {
    if constexpr (SIZE == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voffset, soffset, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, voffset, soffset, 0, 0);
}

template <int FMT, bool DUAL, int MT, int NS, int WV>
__global__ __launch_bounds__(64 * WV) void gemm_ring_kernel(GArgs a, int split) {
    constexpr int NT = 64 * WV;                      // threads
    constexpr int BM = ring_bm<MT, WV>();
    constexpr int XB = BM * 64;                      // bytes of one x half tile (BM rows x 32 BF16)
    constexpr int WRB = ring_w_row_bytes<FMT>();     // raw weight bytes per row and stage
    constexpr int WB = BN * WRB;                     // raw weight bytes per matrix and stage
    constexpr int NWM = DUAL ? 2 : 1;
    constexpr int SLOT = 2 * XB + NWM * WB;
    constexpr bool CONV = FMT != FMT_BF16;
    constexpr int WCB = BN * 64;                     // one converted BF16 weight tile
    constexpr int GW = ring_w_granule<FMT, WV>();    // weight copy granule
    constexpr int NIX = XB / 1024;                   // 1 KB copies per x half
    constexpr int NIW = WB / (64 * GW);              // copies per weight matrix
    constexpr int D = 2 * NIX / WV + NWM * NIW / WV; // copies per wave and stage
    constexpr int CPT = BN * 32 / NT;                // codes each thread converts per matrix and stage
    static_assert(NIX % WV == 0 && NIW % WV == 0, "copies must split evenly over the waves");
    static_assert(CPT == 8 || CPT == 16, "8 or 16 codes per converting thread");
    static_assert(NS >= 4, "the converted weights trail the ring by one stage");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *ring = smem;
    uint8_t *wcv = smem + NS * SLOT;  // CONV: [3][NWM] converted tiles

    int n0, m0;
    tile_of((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, n0, m0, BM);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wm = (wave >> 1) * 32 * MT, wn = (wave & 1) * 64;
    // split 0: all of K; 1: chunk blockIdx.z; 2: half blockIdx.z of a single
    // matrix's chunks (the first hc chunks, then the rest).
    const int hc = (a.nchunks + 1) / 2;
    const int kbeg = split == 1 ? blockIdx.z * a.chunk : split == 2 && blockIdx.z ? hc * a.chunk : 0;
    const int kend = split == 1 ? min(a.K, kbeg + a.chunk) : split == 2 && !blockIdx.z ? min(a.K, hc * a.chunk) : a.K;
    const int nst = (kend - kbeg) / BK;

    const __amdgpu_buffer_rsrc_t rxh = __builtin_amdgcn_make_buffer_rsrc((void *)a.xh, (short)0, a.M * a.K * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rxl = __builtin_amdgcn_make_buffer_rsrc((void *)a.xl, (short)0, a.M * a.K * 2, 0x00020000);
    const int wbytes = (int)((size_t)a.N * a.stride);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)a.w, (short)0, wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw2 =
        __builtin_amdgcn_make_buffer_rsrc((void *)(DUAL ? a.w2 : a.w), (short)0, wbytes, 0x00020000);

    // Per-lane source offsets of this wave's copies (fixed for the launch):
    // x copy q covers rows 16q..16q+15, lane -> row 16q + lane/4 and 16-byte
    // chunk swz(row, lane % 4) of the stage's 32 columns.
    int xoff[NIX / WV], woff[NIW / WV];
#pragma unroll
    for (int i = 0; i < NIX / WV; ++i) {
        const int q = wave + WV * i, r = 16 * q + (lane >> 2);
        const int m = min(m0 + r, a.M - 1);  // rows past M feed only unstored outputs
        xoff[i] = (m * a.K + 8 * swz(r, lane & 3)) * 2;
    }
#pragma unroll
    for (int i = 0; i < NIW / WV; ++i) {
        const int q = wave + WV * i;
        int r, byte;
        if constexpr (FMT == FMT_BF16) { r = 16 * q + (lane >> 2); byte = 16 * swz(r, lane & 3); }
        else if constexpr (FMT == FMT_Q8 && GW == 16) { r = 32 * q + (lane >> 1); byte = 16 * (lane & 1); }
        else if constexpr (FMT == FMT_Q8) { r = 8 * q + (lane >> 3); byte = 4 * (lane & 7); }
        else { r = 16 * q + (lane >> 2); byte = 4 * (lane & 3); }
        const int n = min(n0 + r, a.N - 1);
        woff[i] = n * (int)a.stride + byte;
    }
    // Stage st's copies into ring slot st % NS (stages past the range re-read
    // the last one into a free slot, so every wave issues the same count).
    auto issue = [&](int st) {
        const int k0 = kbeg + min(st, nst - 1) * BK;
        uint8_t *slot = ring + (st % NS) * SLOT;
        const int kx = k0 * 2;
        const int kw = FMT == FMT_BF16 ? k0 * 2 : FMT == FMT_Q8 ? k0 : k0 / 2;
#pragma unroll
        for (int i = 0; i < NIX / WV; ++i) {
            const int q = wave + WV * i;
            buf_to_lds<16>(rxh, slot + 1024 * q, xoff[i], kx);
            buf_to_lds<16>(rxl, slot + XB + 1024 * q, xoff[i], kx);
        }
#pragma unroll
        for (int i = 0; i < NIW / WV; ++i) {
            const int q = wave + WV * i;
            buf_to_lds<GW>(rw, slot + 2 * XB + 64 * GW * q, woff[i], kw);
            if constexpr (DUAL)
                buf_to_lds<GW>(rw2, slot + 2 * XB + WB + 64 * GW * q, woff[i], kw);
        }
    };
    // Q8/Q4: stage st's codes -> BF16 tile(s) wcv[st % 3], thread t: row
    // t / (32 / CPT), codes CPT (t % (32 / CPT)) .. + CPT - 1, written in the
    // swizzled layout the MFMA reads.
    // The raw codes are read by inline assembly: the compiler, which cannot
    // tell these reads from the ring's in-flight copies, would otherwise wait
    // for every copy (all NS stages) before them. The copies they need were
    // awaited explicitly.
    auto convert = [&](int st) {
        constexpr int TPR = 32 / CPT;  // threads per row
        constexpr int RB = FMT == FMT_Q8 ? CPT : CPT / 2;  // raw bytes per thread
        const uint8_t *slot = ring + (st % NS) * SLOT + 2 * XB;
        const int row = threadIdx.x / TPR, h = threadIdx.x % TPR;
        // (Each read waits for its data inside its own asm statement, so no
        // use of the result can be scheduled ahead of the wait.)
        u32x4 rv[NWM];
#pragma unroll
        for (int mi = 0; mi < NWM; ++mi) {
            const uint32_t addr = (uint32_t)(uintptr_t)(slot + mi * WB + row * WRB + RB * h);
            if constexpr (RB == 16) {
                asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(rv[mi]) : "v"(addr) : "memory");
            } else if constexpr (RB == 8) {
                uint2 t;
                asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(t) : "v"(addr) : "memory");
                rv[mi] = u32x4{t.x, t.y, 0u, 0u};
            } else {
                uint32_t t;
                asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(t) : "v"(addr) : "memory");
                rv[mi] = u32x4{t, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int mi = 0; mi < NWM; ++mi) {
            float f[CPT];
            if constexpr (FMT == FMT_Q8) {
                const u32x4 v = rv[mi];
#pragma unroll
                for (int q = 0; q < CPT; ++q) f[q] = (float)(int)(int8_t)(v[q >> 2] >> (8 * (q & 3)));
            } else {
                // 16 x code: each nibble moved to the top of a byte, read as
                // int8 in one instruction (exact in BF16; the chunk sums are
                // scaled back by 1/16, exactly).
#pragma unroll
                for (int h2 = 0; h2 < CPT / 8; ++h2) {
                    const uint32_t wd = rv[mi][h2];
                    const uint32_t ev = (wd << 4) & 0xF0F0F0F0u, od = wd & 0xF0F0F0F0u;
                    f[8 * h2 + 0] = sbyte_f32<0>(ev);
                    f[8 * h2 + 1] = sbyte_f32<0>(od);
                    f[8 * h2 + 2] = sbyte_f32<1>(ev);
                    f[8 * h2 + 3] = sbyte_f32<1>(od);
                    f[8 * h2 + 4] = sbyte_f32<2>(ev);
                    f[8 * h2 + 5] = sbyte_f32<2>(od);
                    f[8 * h2 + 6] = sbyte_f32<3>(ev);
                    f[8 * h2 + 7] = sbyte_f32<3>(od);
                }
            }
            uint8_t *dst = wcv + ((st % 3) * NWM + mi) * WCB + row * 64;
#pragma unroll
            for (int c = 0; c < CPT / 8; ++c) {
                bf16x8 b;
#pragma unroll
                for (int e = 0; e < 8; ++e) b[e] = (__bf16)f[8 * c + e];
                *(bf16x8 *)(dst + 16 * swz(row, (CPT / 8) * h + c)) = b;
            }
        }
    };

    // th: a single matrix's first-half total while the second half runs
    // (folding in registers over all of K).
    f32x16 acc[MT][2], acc2[DUAL ? MT : 1][2], tot[MT][2], tot2[DUAL ? MT : 1][2], th[DUAL ? 1 : MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            tot[i][j] = f32x16{};
            if constexpr (DUAL) tot2[i][j] = f32x16{};
            else th[i][j] = f32x16{};
        }

#pragma unroll
    for (int st = 0; st < NS - 2; ++st) issue(st);
    if constexpr (CONV) {
        __builtin_amdgcn_s_waitcnt(vm_wait_imm(D * (NS - 3)));
        __builtin_amdgcn_s_barrier();
        convert(0);
    }
    const int cs = a.chunk / BK;  // stages per accumulation chunk
    const bool halves = !DUAL && !split && hc < a.nchunks;
    for (int c0 = 0; c0 < nst; c0 += cs) {
        const int c1 = min(c0 + cs, nst);
        // The second half begins: th = t, t = 0.
        const bool half_start = halves && c0 == hc * cs;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[i][j] = f32x16{};
                if constexpr (DUAL) {
                    acc2[i][j] = f32x16{};
                } else if (half_start) {
                    th[i][j] = tot[i][j];
                    tot[i][j] = f32x16{};
                }
            }
        for (int st = c0; st < c1; ++st) {
            issue(st + NS - 2);
            // This wave's copies of stage st (and, converting, st + 1) have
            // landed once only the later stages' copies are pending; after
            // the barrier every wave's have, and the tile converted in the
            // previous iteration is visible.
            __builtin_amdgcn_s_waitcnt(vm_wait_imm(D * (CONV ? NS - 3 : NS - 2)));
            __builtin_amdgcn_s_waitcnt(vm_wait_imm(63) & ~(0xF << 8));  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            const uint8_t *xs = ring + (st % NS) * SLOT;
            const uint8_t *wt = CONV ? wcv + (st % 3) * NWM * WCB : xs + 2 * XB;
            const uint8_t *wt2 = wt + (CONV ? WCB : WB);
            // Every fragment of the stage is read before the first MFMA, so
            // the LDS latency is paid once per stage, not once per k-step.
            constexpr int KS = BK / 16;
            bf16x8 ah[KS][MT], al[KS][MT], bw[KS][2], bw2[KS][DUAL ? 2 : 1];
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                const int c = 2 * k + (lane >> 5);
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const int r = wm + 32 * i + (lane & 31);
                    ah[k][i] = *(const bf16x8 *)(xs + r * 64 + 16 * swz(r, c));
                    al[k][i] = *(const bf16x8 *)(xs + XB + r * 64 + 16 * swz(r, c));
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int r = wn + 32 * j + (lane & 31);
                    bw[k][j] = *(const bf16x8 *)(wt + r * 64 + 16 * swz(r, c));
                    if constexpr (DUAL) bw2[k][j] = *(const bf16x8 *)(wt2 + r * 64 + 16 * swz(r, c));
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
            for (int k = 0; k < KS; ++k)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[k][i], bw[k][j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[k][i], bw[k][j], acc[i][j], 0, 0, 0);
                        if constexpr (DUAL) {
                            acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[k][i], bw2[k][j], acc2[i][j], 0, 0, 0);
                            acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[k][i], bw2[k][j], acc2[i][j], 0, 0, 0);
                        }
                    }
            // Stage st + 1's codes, converted while this stage's MFMAs drain
            // (measured 2-7 % faster than converting before them).
            if constexpr (CONV) {
                if (st + 1 < nst) convert(st + 1);
            }
        }
        // Chunk end: t += c (Q4: c = acc / 16, exactly).
        constexpr float cs16 = FMT == FMT_Q4 ? 0.0625f : 1.0f;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                tot[i][j] += FMT == FMT_Q4 ? acc[i][j] * cs16 : acc[i][j];
                if constexpr (DUAL) tot2[i][j] += FMT == FMT_Q4 ? acc2[i][j] * cs16 : acc2[i][j];
            }
    }
    // Drain the copies of stages past the range before the block exits.
    __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
    if (!split) {
        if constexpr (!DUAL) {
            if (halves) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) tot[i][j] = th[i][j] + tot[i][j];
            }
        }
        epilogue_tile<DUAL, MT>(a, tot, tot2, m0 + wm, n0 + wn, lane);
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        if (n >= a.N) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int m = m0 + wm + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                if (m >= a.M) continue;
                const size_t o = ((size_t)blockIdx.z * a.M + m) * a.N + n;
                a.ws[o] = tot[i][j][q];
                if constexpr (DUAL) a.ws[(size_t)a.nstored * a.M * a.N + o] = tot2[i][j][q];
            }
    }
}

template <int FMT, bool DUAL, int MT, int WV = 4>
int launch_ring(const GArgs &a, int split, hipStream_t s) {
    constexpr int NS = 4, BM = ring_bm<MT, WV>();
    constexpr size_t lds = ring_lds_bytes<FMT, DUAL, MT, NS, WV>();
    static bool attr_set = false;
    if (!attr_set) {
        CHIP_CHECK(hipFuncSetAttribute((const void *)gemm_ring_kernel<FMT, DUAL, MT, NS, WV>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set = true;
    }
    const dim3 grid((a.N + BN - 1) / BN * ((a.M + BM - 1) / BM), 1, split ? a.nstored : 1);
    hipLaunchKernelGGL((gemm_ring_kernel<FMT, DUAL, MT, NS, WV>), grid, dim3(64 * WV), lds, s, a, split);
    CHIP_CHECK(hipGetLastError());
    if (split && !a.defer) {
        const size_t MN = (size_t)a.M * a.N;
        hipLaunchKernelGGL((gemm_reduce_kernel<DUAL>), dim3((unsigned)((MN + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, s, a);
        CHIP_CHECK(hipGetLastError());
    }
    return 0;
}

// Folds the stored sums (a.nstored per output: every chunk's, or a single
// matrix's two halves) in the GEMM's association and applies the epilogue:
// the same bits as the in-register fold. Dual: left to right (t = 0;
// t += c_z); single matrix: the first ceil(n / 2) left to right, the rest
// left to right, then the two added.
template <bool DUAL>
__global__ __launch_bounds__(kThreads) void gemm_reduce_kernel(GArgs a) {
    const size_t MN = (size_t)a.M * a.N;
    const size_t e = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= MN) return;
    const int n = a.nstored, hs = DUAL ? n : (n + 1) / 2;
    // Eight stored sums (of each matrix) loaded at a time, folded in order.
    float v = 0.f, v2 = 0.f, u = 0.f;
    for (int z0 = 0; z0 < n; z0 += 8) {
        float t[8], t2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool in = z0 + j < n;
            t[j] = in ? a.ws[(size_t)(z0 + j) * MN + e] : 0.f;
            if constexpr (DUAL) t2[j] = in ? a.ws[((size_t)n + z0 + j) * MN + e] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (z0 + j < hs) v += t[j];
            else if (z0 + j < n) v2 += t[j];
            if constexpr (DUAL)
                if (z0 + j < n) u += t2[j];
        }
    }
    if (!DUAL && hs < n) v = v + v2;
    epilogue<DUAL>(a, (int)(e / a.N), (int)(e % a.N), v, u);
}

template <int FMT, bool DUAL, int MT>
int launch_mt(const GArgs &a, bool split, hipStream_t s) {
    constexpr int BM = 64 * MT;
    const dim3 grid((a.N + BN - 1) / BN * ((a.M + BM - 1) / BM), 1, split ? a.nchunks : 1);
    if (a.xh) hipLaunchKernelGGL((gemm_kernel<FMT, DUAL, MT, true>), grid, dim3(kThreads), 0, s, a, split ? 1 : 0);
    else hipLaunchKernelGGL((gemm_kernel<FMT, DUAL, MT, false>), grid, dim3(kThreads), 0, s, a, split ? 1 : 0);
    CHIP_CHECK(hipGetLastError());
    if (split && !a.defer) {
        const size_t MN = (size_t)a.M * a.N;
        hipLaunchKernelGGL((gemm_reduce_kernel<DUAL>), dim3((unsigned)((MN + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, s, a);
        CHIP_CHECK(hipGetLastError());
    }
    return 0;
}

// Whether `blocks` blocks of one per CU keep at least 3/4 of the CU slots of
// their rounds busy (288 blocks on 256 CUs: a second round of 32 does not).
bool fills_rounds(long blocks, long cus) {
    const long rounds = (blocks + cus - 1) / cus;
    return blocks >= 1 && 4 * blocks >= 3 * rounds * cus;
}
// 8-wave blocks of 128 tokens x 128 rows: their tiles cover at least 7/8 of
// the CUs and fill their rounds.
bool gemm_w8(int N, int M) {
    const long tiles128 = (long)((N + BN - 1) / BN) * ((M + 127) / 128), cus = device_cus();
    return tiles128 * 8 >= cus * 7 && fills_rounds(tiles128, cus);
}
// Whether a single matrix's GEMM runs as two chunk halves on 8-wave blocks:
// two blocks per 128-token tile fill 95-100 % of the CUs in one round, and
// it has more than one chunk.
bool gemm_halves_split(int N, int M, int nchunks) {
    const long tiles128 = (long)((N + BN - 1) / BN) * ((M + 127) / 128), cus = device_cus();
    return nchunks > 1 && 2 * tiles128 * 20 >= cus * 19 && 2 * tiles128 <= cus;
}

template <int FMT>
int launch_fmt(GArgs a, bool dual, size_t ws_floats, hipStream_t s, bool &split_out, int &stored_out) {
    const long n_tiles = (a.N + BN - 1) / BN;
    const long tiles128 = n_tiles * ((a.M + 127) / 128), tiles64 = n_tiles * ((a.M + 63) / 64);
    const long cus = device_cus();
    // Many tiles: fold in registers. Few tiles: split-K over the chunks when
    // the workspace holds them.
    const bool split = a.nchunks > 1 && tiles64 < cus && a.ws &&
                       ws_floats >= gemm_workspace_floats(a.N, a.K, a.M, dual);
    split_out = split;
    a.nstored = a.nchunks;
    stored_out = a.nstored;
    // Pre-split x with K a multiple of the stage and 32-bit buffer offsets:
    // the ring kernel (weights copied 16 bytes at a time, Q4 4 at a time).
    const int galign = FMT == FMT_Q4 ? 4 : 16;
    const bool ring = a.xh && a.K % BK == 0 && a.stride % galign == 0 &&
                      ((uintptr_t)a.w % galign) == 0 && (!dual || ((uintptr_t)a.w2 % galign) == 0) &&
                      (size_t)a.M * a.K * 2 < (1ull << 31) && (size_t)a.N * a.stride < (1ull << 31);
    // 8-wave blocks of 128 tokens x 128 rows where those tiles cover at
    // least 7/8 of the CUs: each converted weight tile and each x tile in
    // LDS then serves twice the MFMAs of a 4-wave 64-token block, with the
    // same waves per CU (one 8-wave block against two 4-wave ones). Measured
    // at 1,024 tokens: BF16 4096x4096 358 -> 418, 4096x14336 310 -> 402,
    // 3584x18944 298 -> 370 TFLOP/s; Llama-3-8B Q4 512-row prefill 17.2K ->
    // 18.6K tok/s (mostly the dual gate/up, which before took 128-token tiles
    // on 4 waves), Qwen2-7B 1,024-row 18.2K -> 19.2K; the same bits. Where
    // the 128-token tiles cover only half the CUs (4096 rows at 512 tokens:
    // 128 tiles), 4-wave 64-token blocks are faster (307 vs 242 TFLOP/s).
    if (ring && !split && gemm_w8(a.N, a.M))
        return dual ? launch_ring<FMT, true, 1, 8>(a, 0, s) : launch_ring<FMT, false, 1, 8>(a, 0, s);
    // A single matrix whose 128-token tiles cover half the CUs (4,096 rows
    // at 512 tokens: 128 tiles): its two chunk halves on separate 8-wave
    // blocks, the half sums folded by the reader.
    if (ring && !split && !dual && gemm_halves_split(a.N, a.M, a.nchunks) && a.ws &&
        ws_floats >= 2 * (size_t)a.M * a.N) {
        split_out = true;
        a.nstored = stored_out = 2;
        return launch_ring<FMT, false, 1, 8>(a, 2, s);
    }
    const int sp = split ? 1 : 0;
    if (ring) return dual ? launch_ring<FMT, true, 1>(a, sp, s) : launch_ring<FMT, false, 1>(a, sp, s);
    // Otherwise (K not a multiple of the stage, x not pre-split, or operands
    // beyond the buffer loads' 32-bit offsets): the register-staged kernel.
    if (dual) return launch_mt<FMT, true, 1>(a, split, s);
    if (!split && tiles128 >= cus) return launch_mt<FMT, false, 2>(a, false, s);
    return launch_mt<FMT, false, 1>(a, split, s);
}

// x -> hi = bf16(x), lo = bf16(x - hi), 4 elements per thread.
__global__ __launch_bounds__(kThreads) void split_bf16_kernel(const float *x, size_t n, uint16_t *xh, uint16_t *xl) {
    const size_t i = ((size_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i >= n) return;
    if (i + 4 <= n) {
        const f32x4 v = *(const f32x4 *)(x + i);
        uint16_t h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const __bf16 hb = (__bf16)v[q];
            h[q] = __builtin_bit_cast(uint16_t, hb);
            l[q] = __builtin_bit_cast(uint16_t, (__bf16)(v[q] - (float)hb));
        }
        *(uint2 *)(xh + i) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
        *(uint2 *)(xl + i) = make_uint2(pack2(l[0], l[1]), pack2(l[2], l[3]));
    } else {
        for (size_t q = i; q < n; ++q) {
            const __bf16 hb = (__bf16)x[q];
            xh[q] = __builtin_bit_cast(uint16_t, hb);
            xl[q] = __builtin_bit_cast(uint16_t, (__bf16)(x[q] - (float)hb));
        }
    }
}

}  // namespace

int launch_split_bf16(const float *x, size_t n, uint16_t *xh, uint16_t *xl, hipStream_t s) {
    if (n == 0) return 0;
    if (!x || !xh || !xl || ((uintptr_t)x % 16) || ((uintptr_t)xh % 8) || ((uintptr_t)xl % 8))
        return fail("HIP backend: split needs 16-byte aligned input and 8-byte aligned halves.");
    const size_t threads = (n + 3) / 4;
    hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       x, n, xh, xl);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

// Accumulation chunk depth, a function of K alone (so a token's bits never
// depend on the call's token count): at least 256 and K / 16; K up to 1024
// in three chunks instead (K = 896: 320 + 320 + 256 rather than 3 x 256 +
// 128; the split-K blocks of a 128-token chunk then fit the chip in one
// round: Qwen2-0.5B prefill 61.0K -> 65.0K tok/s; two chunks 63.0K, four
// equal 61.0K, one 49.9K).
int gemm_chunk_depth(int K) {
    const int want = K <= 1024 ? (K + 2) / 3 : std::max(256, (K + 15) / 16);
    return (want + BK - 1) / BK * BK;
}

size_t gemm_workspace_floats(size_t N, size_t K, size_t M, bool dual) {
    const int chunk = gemm_chunk_depth((int)K);
    const size_t nchunks = (K + chunk - 1) / chunk;
    if (nchunks <= 1) return 0;
    return nchunks * M * N * (dual ? 2 : 1);
}

size_t gemm_split_workspace_floats(size_t N, size_t K, size_t m_max, bool dual) {
    // The per-chunk split runs only while 64-token tiles leave CUs idle; the
    // two-half split (single matrices) while two blocks per 128-token tile
    // fit the CUs once.
    const size_t n_tiles = (N + BN - 1) / BN, cus = (size_t)device_cus();
    const size_t m_split = 64 * ((cus + n_tiles - 1) / n_tiles);
    size_t need = gemm_workspace_floats(N, K, std::min(m_max, m_split), dual);
    const int chunk = gemm_chunk_depth((int)K);
    if (!dual && (K + chunk - 1) / chunk > 1)
        need = std::max(need, 2 * std::min(m_max, 128 * (cus / (2 * n_tiles))) * N);
    return need;
}

int launch_gemm(const GemmJob &job, hipStream_t s) {
    const WMat &w = job.w;
    if (job.n == 0) return 0;
    if (!w.base || !job.x || w.rows == 0 || w.cols == 0) return fail("HIP backend: gemm needs a weight and an input.");
    if (w.rows > (size_t)INT32_MAX || w.cols > (size_t)INT32_MAX || job.n > 65535u * 64u)
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
    if (!job.yh != !job.yl) return fail("HIP backend: gemm output halves need both BF16 buffers or neither.");
    a.yh = dual ? job.yh : nullptr;
    a.yl = dual ? job.yl : nullptr;
    a.defer = job.deferred && !dual ? 1 : 0;
    if (job.deferred) *job.deferred = 0;
    a.epi = job.epi;
    a.chunk = gemm_chunk_depth(a.K);
    a.nchunks = (a.K + a.chunk - 1) / a.chunk;
    a.ws = job.ws;
    a.vec_x = (a.K % 4) == 0 && ((uintptr_t)job.x % 16) == 0;
    // Pre-split halves are used when every 8-element chunk is 16-byte aligned.
    const bool pre = job.xh && job.xl && a.K % 8 == 0 && ((uintptr_t)job.xh % 16) == 0 && ((uintptr_t)job.xl % 16) == 0;
    a.xh = pre ? job.xh : nullptr;
    a.xl = pre ? job.xl : nullptr;
    const uintptr_t p1 = (uintptr_t)a.w, p2 = dual ? (uintptr_t)a.w2 : p1;
    if (w.fmt == FMT_BF16) a.vec_w = a.stride % 16 == 0 && p1 % 16 == 0 && p2 % 16 == 0 && a.K % 8 == 0;
    else if (w.fmt == FMT_Q8) a.vec_w = a.stride % 16 == 0 && p1 % 16 == 0 && p2 % 16 == 0 && a.K % 16 == 0;
    else a.vec_w = 0;
    if (w.fmt == FMT_Q4 && (a.stride % 4 != 0 || p1 % 4 != 0 || p2 % 4 != 0))
        return fail("HIP backend: Q4 rows must be 4-byte aligned.");
    bool split = false;
    int stored = 0, rc = -1;
    switch (w.fmt) {
        case FMT_BF16: rc = launch_fmt<FMT_BF16>(a, dual, job.ws_floats, s, split, stored); break;
        case FMT_Q8: rc = launch_fmt<FMT_Q8>(a, dual, job.ws_floats, s, split, stored); break;
        case FMT_Q4: rc = launch_fmt<FMT_Q4>(a, dual, job.ws_floats, s, split, stored); break;
        default: return fail("HIP backend: unknown weight format.");
    }
    if (rc == 0 && a.defer && split) *job.deferred = stored;
    return rc;
}

}  // namespace chip
