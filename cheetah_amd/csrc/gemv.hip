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
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <numeric>
#include <type_traits>
#include <vector>

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

// ---------------------------------------------------------------------------
// Aligned-unit GEMV: every row is streamed as 16-byte units from its
// 16-byte-aligned-down start, even when the reference layout only aligns rows
// to 4 bytes (Q4 rows of 2052 / 7172 bytes, Q8 rows of K rounded up to 4).
// Bytes of a unit that lie outside the row (the previous row's tail or the
// scale head before it; padding after it) meet zeros: x sits in LDS between
// 32 zero floats on each side and the unit's x window is shifted by the row's
// misalignment, which is a multiple of 4 floats (Q8: delta, Q4: 2 * delta for
// delta in {0, 4, 8, 12}), so every x read stays a 16-byte LDS read. Rows of
// one group share their misalignment: the R rows of a group are P apart,
// P = 16 / gcd(stride mod 16, 16). The grid is persistent (occupancy-sized),
// so each block stages x once and streams many row groups.
// ---------------------------------------------------------------------------
constexpr int kPad = 32;  // zero floats before and after x in LDS


// Q4 x with two rows per wave (one matrix) sits in LDS with 4 spare floats
// after every 32 elements (one unit): lane i's unit starts 128 bytes after
// lane i - 1's, so unpadded every other lane's 16-byte reads fall on the same
// 4 banks; at a 144-byte stride 16 consecutive lanes hit 16 distinct groups
// of 4 banks. Element e (>= -kPad, the zeros before x) is at
// x_addr(e) = e + ((e >> 5) << 2); a 16-byte read of 4 elements never
// straddles a gap. Measured: Q4 4096x14336 10.9 -> 9.5 us, 4096^2 6.0 -> 5.7;
// with the dual gate/up or Q8/BF16 the extra address
// arithmetic costs more than the conflicts (x stays unpadded: xl = 0).
__host__ __device__ constexpr int x_shift_log2(int fmt, int rows, bool dual) {
    return fmt == FMT_Q4 && rows == 2 && !dual ? 5 : 0;
}
__host__ __device__ constexpr int x_addr(int e, int xl) { return xl ? e + ((e >> xl) << 2) : e; }
// Floats of padded x from its first element to past its trailing zeros.
__host__ __device__ constexpr int x_span(int K, int xl) { return x_addr(K + kPad, xl) + 4; }

// Dynamic LDS of the aligned kernel: x (padded per x_shift_log2) and the
// norm gain as BF16.
inline size_t aligned_lds(int K, bool norm, int xl) {
    return (size_t)(kPad + x_span(K, xl)) * sizeof(float) + (norm ? (size_t)K * 2 + 16 : 0);
}
// The largest of those over the instantiations a launch may pick.
inline size_t aligned_lds_max(int K, bool norm) { return aligned_lds(K, norm, 5); }
// Buffer descriptor word 3 for raw (untyped, unswizzled) buffer access on
// gfx9-family chips, and the non-temporal cache policy bit of a buffer load.
constexpr int kBufferDword3 = 0x00020000;
constexpr int kBufferNT = 2;
// 16 bytes per lane from global memory into LDS at lds + 16 * lane (lds the
// same in every lane). The copy takes its LDS base from m0, which the
// compiler reserves, so the old value is saved and restored around it; the
// compiler does not see the copy (the caller waits for it with
// wait_vm_but), so its later LDS reads do not wait for the weight loads in
// flight, as they would after the compiler's own global_load_lds builtin.
__device__ __forceinline__ void lds_dma16(const void *g, const void *lds) {
    const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(l)
        : "memory");
}
// Waits until at most N of this wave's vector memory operations are in
// flight (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm_but() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

constexpr int kAThreads = 512;  // at most 8 waves share one x staging
constexpr int kAWaves = kAThreads / 64;

// One aligned GEMV (see the file head) as the work of one block: `bid` of
// `nblk` blocks of kAThreads threads.
template <int FMT, int R, int KS, bool NORM, bool DUAL, int UNROLL>
struct AlignedGemv {
    using U = Unit<FMT, 16>;
    static constexpr int E = U::E;
    static constexpr int D = 4;
    static constexpr int STEP = 64 * KS * UNROLL;
    static constexpr int NM = DUAL ? 2 : 1;
    static constexpr int XL = x_shift_log2(FMT, R, DUAL);
    static constexpr int NLOADS = UNROLL * NM * R;  // vector loads of one batch
    typedef uint32_t Batch[UNROLL][NM][R][D];

    const Args &a;
    const int P;
    int tid, lane, wave, sub, klane, K, row_bytes, groups, g, gstride, iters;
    const uint8_t *ap[NM][R];  // aligned-down row starts
    // One buffer descriptor per row over its nfull whole units: a load past
    // them returns zeros and moves no memory, so every batch load is issued
    // unconditionally and the compiler can wait on exactly the older batch.
    __amdgpu_buffer_rsrc_t rs[NM][R];
    int row_of[R];
    int shift = 0, nfull = 0;
    bool gvalid = false, first_issued = false;
    Batch A, B;

    __device__ __forceinline__ AlignedGemv(const Args &args, int phases, int bid, int nblk) : a(args), P(phases) {
        tid = threadIdx.x;
        lane = tid & 63;
        // Wave-uniform, so the row pointers below live in scalar registers
        // and make buffer descriptors without a per-lane loop.
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        constexpr int gpb = kAWaves / KS;  // row groups per block
        sub = wave % KS;
        klane = sub * 64 + lane;
        K = a.K;
        row_bytes = FMT == FMT_Q4 ? (K + 1) / 2 : (FMT == FMT_Q8 ? K : 2 * K);
        groups = (a.rows + R * P - 1) / (R * P) * P;
        // The block's waves take consecutive row groups (neighbouring rows:
        // measured faster than spreading them over the blocks, Q4 gate/up
        // of a Llama-3-8B layer 18.8 vs 19.3 us).
        g = bid * gpb + wave / KS;
        gstride = nblk * gpb;
        // Every wave of the block runs the same number of iterations (the
        // cross-wave K reduction synchronizes the block).
        iters = (groups - bid * gpb + gstride - 1) / gstride;
    }

    __device__ __forceinline__ void set_group(int gg) {
        const int blk = gg / P, ph = gg % P;
        const int row0 = blk * R * P + ph;
        // The last block of rows can leave phases without a first row: such
        // a group loads nothing and stores nothing.
        gvalid = row0 < a.rows;
        if (!gvalid) {
            nfull = 0;
            shift = 0;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                row_of[r] = a.rows;
                ap[0][r] = a.w;
                if constexpr (DUAL) ap[1][r] = a.w2;
            }
            return;
        }
        const uintptr_t p0 = (uintptr_t)(a.w + (size_t)row0 * a.stride);
        const int delta = (int)(p0 & 15);
        shift = delta * E / 16;
        nfull = (delta + row_bytes) / 16;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r * P;
            row_of[r] = row;
            const int rr = row < a.rows ? row : row0;  // same misalignment, always in bounds
            ap[0][r] = a.w + (size_t)rr * a.stride - delta;
            if constexpr (DUAL) ap[1][r] = a.w2 + (size_t)rr * a.stride - delta;
        }
    }
    __device__ __forceinline__ void set_rsrc() {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
                rs[m][r] = __builtin_amdgcn_make_buffer_rsrc((void *)ap[m][r], (short)0, nfull * 16, kBufferDword3);
    }
    __device__ __forceinline__ void load_batch(Batch &buf, int u0) {
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) {
            const int u = u0 + 64 * KS * i;
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const u32x4 v = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[m][r], u * 16, 0, kBufferNT));
                    buf[i][m][r][0] = v[0];
                    buf[i][m][r][1] = v[1];
                    buf[i][m][r][2] = v[2];
                    buf[i][m][r][3] = v[3];
                }
        }
    }
    // The first row group's first batch (issued at most once).
    __device__ __forceinline__ void start() {
        if (first_issued) return;
        first_issued = true;
        if (g < groups) {
            set_group(g);
            set_rsrc();
            load_batch(A, klane);
        }
    }
    // Waits until this wave's operations issued before start() are done,
    // leaving the first batch in flight.
    __device__ __forceinline__ void wait_before_first() {
        if (g < groups) wait_vm_but<NLOADS>();
        else wait_vm_but<0>();
    }

    // Zero padding, then x (and the norm gain) as direct global->LDS copies.
    // Padded x: lanes in groups of nine, eight 16-byte pieces of one
    // 32-element block and one that fills the 16-byte gap after it (never
    // read), 7 blocks per instruction. Returns whether the gain went to LDS.
    __device__ __forceinline__ bool stage_x(float *xs_all) {
        float *xs = xs_all + kPad;
        for (int i = tid; i < kPad; i += kAThreads) {
            xs_all[i] = 0.f;
            xs[x_addr(K + i, XL)] = 0.f;
        }
        float *gs = xs + x_span(K, XL);  // gain as floats-of-bf16-pairs (NORM only)
        const bool dma_x = ((uintptr_t)a.x % 16) == 0 && (K % 4) == 0;
        const bool dma_g = NORM && ((uintptr_t)a.gain % 16) == 0 && (K % 8) == 0;
        if (dma_x) {
            if constexpr (XL != 0) {
                static_assert(XL == 5, "padded x in 32-element blocks");
                const int j = lane / 9, q = lane % 9;
                for (int c = wave; c * 224 < K; c += kAWaves) {
                    const int blk = c * 224 + 32 * j, f = blk + 4 * (q < 8 ? q : 0);
                    if (lane < 63 && blk < K && f + 4 <= K) lds_dma16(a.x + f, xs + x_addr(c * 224, XL));
                }
            } else {
                for (int c = wave; c * 256 < K; c += kAWaves) {
                    const int f = c * 256 + lane * 4;
                    if (f < K) lds_dma16(a.x + f, xs + c * 256);
                }
            }
        }
        if (dma_g) {
            for (int c = wave; c * 512 < K; c += kAWaves) {
                const int f = c * 512 + lane * 8;
                if (f < K) lds_dma16(a.gain + f, gs + c * 256);
            }
        }
        if (!dma_x)
            for (int i = tid; i < K; i += kAThreads) xs[x_addr(i, XL)] = a.x[i];
        return dma_g;
    }

    // acc += the batch's weights (units u0 + 64 KS i) times x.
    __device__ __forceinline__ void mac_batch(const Batch &cur, int u0, float (&acc)[NM][R], const float *xs) {
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) {
            const int u = u0 + 64 * KS * i;
            // One weight dword at a time: its E/4 x values (Q4 8, Q8 4,
            // BF16 2) are read once and shared by every row. A unit past the
            // row has zero weights (load_batch) and reads the last unit's x:
            // LDS past x + padding holds whatever an earlier kernel left, and
            // 0 * NaN is NaN.
            const int uu = min(u, nfull - 1);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                constexpr int ED = E / 4;
                float xv[ED];
                // Padded Q4 x: dword d's 8 elements uu E - shift + 8 d .. lie
                // in unit uu's block when 8 d >= shift, else in the one
                // before, so their address is 36 uu - shift - 4 + 8 d, plus 4
                // in the former case.
                const int xd = XL ? 36 * uu - shift - 4 + 8 * d + (8 * d >= shift ? 4 : 0) : uu * E - shift + d * ED;
                if constexpr (ED >= 4) {
#pragma unroll
                    for (int q = 0; q < ED / 4; ++q) {
                        const float4 t = *(const float4 *)(xs + xd + 4 * q);
                        xv[4 * q] = t.x;
                        xv[4 * q + 1] = t.y;
                        xv[4 * q + 2] = t.z;
                        xv[4 * q + 3] = t.w;
                    }
                } else {
                    const float2 t = *(const float2 *)(xs + xd);
                    xv[0] = t.x;
                    xv[1] = t.y;
                }
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t word = cur[i][m][r][d];
                        if constexpr (FMT == FMT_Q4) {
                            // Nibbles moved to the top of bytes read as int8
                            // are 16 x the code; each byte converts in one
                            // instruction. acc holds 16 x the sum, in the same
                            // order, so scaling by 1/16 afterwards is exact.
                            const uint32_t ev = (word << 4) & 0xF0F0F0F0u, od = word & 0xF0F0F0F0u;
                            acc[m][r] = fmaf(sbyte_f32<0>(ev), xv[0], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<0>(od), xv[1], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<1>(ev), xv[2], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<1>(od), xv[3], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<2>(ev), xv[4], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<2>(od), xv[5], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<3>(ev), xv[6], acc[m][r]);
                            acc[m][r] = fmaf(sbyte_f32<3>(od), xv[7], acc[m][r]);
                        } else if constexpr (FMT == FMT_Q8) {
#pragma unroll
                            for (int b = 0; b < 4; ++b)
                                acc[m][r] = fmaf((float)(int)(int8_t)(word >> (8 * b)), xv[b], acc[m][r]);
                        } else {
                            acc[m][r] = fmaf(bf16_lo(word), xv[0], acc[m][r]);
                            acc[m][r] = fmaf(bf16_hi(word), xv[1], acc[m][r]);
                        }
                    }
            }
        }
    }

    // After x has landed (the caller waited and passed a block barrier): the
    // fused RMSNorm, the products of every row group of this block, and the
    // epilogue. red: kAWaves floats; kred: kAWaves x NM R floats (LDS).
    __device__ __forceinline__ void finish(float *xs_all, bool dma_g, float *red, float *kred) {
        float *xs = xs_all + kPad;
        if constexpr (NORM) {
            // RMSNorm (ops.rs:646-652): x * (inv * gain), inv = 1/sqrt(mean(x^2)+eps).
            const float *gs = xs + x_span(K, XL);
            float ss = 0.f;
            for (int i = tid; i < K; i += kAThreads) ss = fmaf(xs[x_addr(i, XL)], xs[x_addr(i, XL)], ss);
            ss = wave_sum(ss);
            if (lane == 0) red[wave] = ss;
            __syncthreads();
            float total = 0.f;
#pragma unroll
            for (int w = 0; w < kAWaves; ++w) total += red[w];
            const float inv = 1.0f / sqrtf(total / (float)K + a.eps);
            const uint16_t *gl = (const uint16_t *)gs;
            for (int i = tid; i < K; i += kAThreads)
                xs[x_addr(i, XL)] = xs[x_addr(i, XL)] * (inv * bf16_f32(dma_g ? gl[i] : a.gain[i]));
            __syncthreads();
        }
        for (int it = 0; it < iters; ++it, g += gstride) {
            const bool valid = g < groups && gvalid;
            float acc[NM][R];
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
            if (valid) {
                // Batches alternate between A and B, so no register copy
                // (which would wait for the prefetch) separates a load from
                // its use: batch j+1 streams in while batch j is multiplied.
                // The batch count is wave-uniform; lanes past the row load
                // zeros.
                const int nb = (nfull - sub * 64 + STEP - 1) / STEP;
                int j = 0;
                // (The scheduling barriers keep the compiler from sinking a
                // prefetch below the multiply-adds to save registers.)
                for (; j + 2 <= nb; j += 2) {
                    load_batch(B, klane + (j + 1) * STEP);
                    __builtin_amdgcn_sched_barrier(0);
                    mac_batch(A, klane + j * STEP, acc, xs);
                    load_batch(A, klane + (j + 2) * STEP);
                    __builtin_amdgcn_sched_barrier(0);
                    mac_batch(B, klane + (j + 1) * STEP, acc, xs);
                }
                if (j < nb) mac_batch(A, klane + j * STEP, acc, xs);
                if constexpr (FMT == FMT_Q4) {
#pragma unroll
                    for (int m = 0; m < NM; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[m][r] *= 0.0625f;
                }
                // Elements past the last whole unit (fewer than 16 bytes' worth).
                for (int e = max(nfull * E - shift, 0) + klane; e < K; e += 64 * KS) {
                    const float xv = xs[x_addr(e, XL)];
#pragma unroll
                    for (int m = 0; m < NM; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[m][r] = fmaf(U::element(ap[m][r] + (shift * 16 / E), e), xv, acc[m][r]);
                }
            }
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);
            int orow[R];
#pragma unroll
            for (int r = 0; r < R; ++r) orow[r] = row_of[r];
            // Prefetch the next group's first batch before the epilogue.
            if (g + gstride < groups) {
                set_group(g + gstride);
                set_rsrc();
                load_batch(A, klane);
            }
            if constexpr (KS > 1) {
                if (lane == 0) {
#pragma unroll
                    for (int m = 0; m < NM; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) kred[wave * NM * R + m * R + r] = acc[m][r];
                }
                __syncthreads();
                if (sub == 0) {
#pragma unroll
                    for (int m = 0; m < NM; ++m)
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            float sacc = kred[wave * NM * R + m * R + r];
#pragma unroll
                            for (int k = 1; k < KS; ++k) sacc += kred[(wave + k) * NM * R + m * R + r];
                            acc[m][r] = sacc;
                        }
                }
                __syncthreads();
            }
            if (sub == 0 && valid) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int row = orow[r];
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
};

template <int FMT, int R, int KS, bool NORM, bool DUAL, int UNROLL>
__global__ __launch_bounds__(kAThreads) void gemv_aligned_kernel(Args a, int P) {
    using G = AlignedGemv<FMT, R, KS, NORM, DUAL, UNROLL>;
    extern __shared__ float4 xs_v4[];  // 16-byte aligned
    __shared__ float red[kAWaves];
    __shared__ float kred[kAWaves * G::NM * R];
    float *xs_all = (float *)xs_v4;
    G gm(a, P, (int)blockIdx.x, (int)gridDim.x);
    // x goes first: a wave's loads complete in order, so the wait ends when
    // x has landed while the first weight batch stays in flight.
    const bool dma_g = gm.stage_x(xs_all);
    gm.start();
    gm.wait_before_first();
    __syncthreads();
    gm.finish(xs_all, dma_g, red, kred);
}

// Waves per SIMD the aligned kernel's VGPR count allows (512 per lane,
// granule 8, at most 8).
template <class Kern>
int aligned_waves_per_simd(Kern kern) {
    static std::mutex mu;
    static std::vector<std::pair<const void *, int>> vgprs;
    int regs = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (auto &e : vgprs)
            if (e.first == (const void *)kern) regs = e.second;
        if (regs == 0) {
            hipFuncAttributes attr{};
            regs = hipFuncGetAttributes(&attr, (const void *)kern) == hipSuccess && attr.numRegs > 0 ? attr.numRegs
                                                                                                     : 128;
            vgprs.push_back({(const void *)kern, regs});
        }
    }
    return std::min(8, 512 / ((regs + 7) / 8 * 8));
}

template <int FMT, int R, int KS, bool NORM, bool DUAL, int UNROLL>
int launch_aligned(const Args &a, int P, hipStream_t s) {
    const int groups = (a.rows + R * P - 1) / (R * P) * P;
    const size_t lds = aligned_lds(a.K, NORM, x_shift_log2(FMT, R, DUAL));
    auto kern = gemv_aligned_kernel<FMT, R, KS, NORM, DUAL, UNROLL>;
    // Blocks of 8 waves, as many per CU as the VGPRs and the LDS allow.
    // (Blocks of 7 waves, which fill the 28 slots of a 7-wave-per-SIMD kernel
    // where 8-wave blocks leave 4 idle, measured slower: the Q4 gate/up of
    // a Llama-3-8B layer 20.4 vs 19.0 us.)
    const int per_cu = std::max(1, std::min(4 * aligned_waves_per_simd(kern) / kAWaves,
                                            (int)(device_lds_per_cu() / (lds + 1024))));
    const int gpb = kAWaves / KS;
    const int cap = device_cus() * per_cu;
    const int blocks = std::max(1, std::min((groups + gpb - 1) / gpb, cap));
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kAThreads), lds, s, a, P);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

template <int FMT, int R, bool NORM, bool DUAL, int UNROLL>
int pick_ks_un(const Args &a, int P, int ks, hipStream_t s) {
    switch (ks) {
        case 8: return launch_aligned<FMT, R, 8, NORM, DUAL, UNROLL>(a, P, s);
        case 4: return launch_aligned<FMT, R, 4, NORM, DUAL, UNROLL>(a, P, s);
        case 2: return launch_aligned<FMT, R, 2, NORM, DUAL, UNROLL>(a, P, s);
        default: return launch_aligned<FMT, R, 1, NORM, DUAL, UNROLL>(a, P, s);
    }
}

// Units per lane per iteration (UNROLL). With two, a row of up to ~1,000
// 16-byte units (a 4096-column Q4 row is 128) takes one or two iterations:
// the waves load, then compute, with little to overlap. One unit per
// iteration puts the next unit's loads in flight during the current FMAs:
// measured 3-17 % faster on such rows, 3-14 % slower on 18,944-column BF16 /
// Q8 rows. A lane takes its units in the same order either way (same bits).
template <int FMT, int R, bool NORM, bool DUAL>
int pick_ks(const Args &a, int P, int ks, int n_units, hipStream_t s) {
    if (n_units / ks <= 1024) return pick_ks_un<FMT, R, NORM, DUAL, 1>(a, P, ks, s);
    return pick_ks_un<FMT, R, NORM, DUAL, 2>(a, P, ks, s);
}

// Rows per wave (R) and waves per row group (KS, splitting K), as measured
// on MI355X (slots = 16 waves per CU): one row per wave streams BF16 / Q8
// best. Q4 (twice the elements per byte) gains from sharing each x read
// between rows once there are enough rows to keep the wave slots busy: two
// rows per wave, measured 5-12 % faster than one (dual 14336x4096: 20.1 vs
// 22.0 us). K is split when
// the row groups are too few for the wave slots (Q4: below a quarter of
// them, since its rows share x reads), keeping >= 2 units per lane.
struct AlignedShape {
    int R, ks, unroll;
};
template <int FMT>
AlignedShape aligned_shape(const Args &a) {
    constexpr int E = Unit<FMT, 16>::E;
    const int n_units = (a.K + E - 1) / E;
    const long slots = (long)device_cus() * 16;
    int R = 1;
    // (Four Q4 rows per wave for 6144-row matrices left the grid under one
    // block per CU: 2,474 vs 2,488 tok/s on a 4-layer Llama-3-8B Q4 decode.)
    if (FMT == FMT_Q4 && a.rows >= slots / 2) R = 2;
    const long groups = (a.rows + R - 1) / R;
    const long busy = FMT == FMT_Q4 ? slots / 4 : slots;
    int ks = 1;
    while (ks < 8 && groups * ks < busy && n_units >= 64 * 2 * ks * 2) ks *= 2;
    // Rows of more than 1,024 units per wave are split further (at most 4
    // ways): BF16 3584 x 18944 (Qwen2-7B down_proj) 5,390 GB/s with 2 ways,
    // 5,858 with 4.
    while (ks < 4 && n_units / ks > 1024) ks *= 2;
    return AlignedShape{R, ks, n_units / ks <= 1024 ? 1 : 2};
}

template <int FMT, bool NORM, bool DUAL>
int pick_aligned(const Args &a, int P, hipStream_t s) {
    constexpr int E = Unit<FMT, 16>::E;
    const int n_units = (a.K + E - 1) / E;
    const AlignedShape sh = aligned_shape<FMT>(a);
    if constexpr (FMT == FMT_Q4) {
        if (sh.R == 2) return pick_ks<FMT, 2, NORM, DUAL>(a, P, sh.ks, n_units, s);
    }
    return pick_ks<FMT, 1, NORM, DUAL>(a, P, sh.ks, n_units, s);
}

template <int FMT>
int pick_aligned_mode(const Args &a, int P, bool norm, bool dual, hipStream_t s) {
    if (norm) return dual ? pick_aligned<FMT, true, true>(a, P, s) : pick_aligned<FMT, true, false>(a, P, s);
    return dual ? pick_aligned<FMT, false, true>(a, P, s) : pick_aligned<FMT, false, false>(a, P, s);
}

// ---------------------------------------------------------------------------
// Dword fallback for layouts the aligned kernel does not take (BF16 rows not
// 16-byte aligned: odd widths in small shapes).
// ---------------------------------------------------------------------------
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

template <int FMT, bool NORM, bool DUAL>
int pick_shape(const Args &a, hipStream_t s) {
    constexpr int E = Unit<FMT, 4>::E;
    const int n_units = a.K / E;
    int ks = 1;
    while (ks < 4 && a.rows * ks < 2048 && n_units >= 64 * ks * 2 * 4) ks *= 2;
    if (ks == 4) return launch_t<FMT, 4, 1, 4, NORM, DUAL>(a, s);
    if (ks == 2) return launch_t<FMT, 4, 1, 2, NORM, DUAL>(a, s);
    return launch_t<FMT, 4, 1, 1, NORM, DUAL>(a, s);
}

template <int FMT>
int pick_mode(const Args &a, bool norm, bool dual, hipStream_t s) {
    if (norm) return dual ? pick_shape<FMT, true, true>(a, s) : pick_shape<FMT, true, false>(a, s);
    return dual ? pick_shape<FMT, false, true>(a, s) : pick_shape<FMT, false, false>(a, s);
}

// A job's kernel arguments, and whether (with which row phase count P) the
// aligned kernel takes it.
struct Prepared {
    Args a;
    bool norm, dual, aligned;
    int P;
};
int prepare(const GemvJob &job, Prepared &out) {
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
    const bool norm = job.norm_gain != nullptr;
    // The aligned kernel needs 4-byte-aligned rows whose misalignment is a
    // multiple of 4 x floats (BF16: rows 16-byte aligned), gate and up
    // misaligned alike, and x plus its padding in LDS.
    const uintptr_t b0 = (uintptr_t)a.w;
    const int bpe_mod = w.fmt == FMT_BF16 ? 16 : 4;
    // The aligned-down start of the first row must not precede the buffer.
    const bool aligned_ok = a.stride % bpe_mod == 0 && b0 % bpe_mod == 0 && (uintptr_t)w.base % 16 == 0 &&
                            (!dual || ((uintptr_t)job.w2.base % 16 == 0 && ((uintptr_t)a.w2 - b0) % 16 == 0)) &&
                            aligned_lds_max(a.K, norm) + 256 <= device_max_lds();
    if (w.fmt != FMT_BF16 && w.fmt != FMT_Q8 && w.fmt != FMT_Q4) return fail("HIP backend: unknown weight format.");
    const int sm = (int)(a.stride % 16);
    out = Prepared{a, norm, dual, aligned_ok, sm == 0 ? 1 : 16 / std::gcd(sm, 16)};
    return 0;
}

}  // namespace

int launch_gemv(const GemvJob &job, hipStream_t s) {
    Prepared p;
    CHIP_TRY(prepare(job, p));
    const Args &a = p.a;
    if (p.aligned) {
        switch (job.w.fmt) {
            case FMT_BF16: return pick_aligned_mode<FMT_BF16>(a, p.P, p.norm, p.dual, s);
            case FMT_Q8: return pick_aligned_mode<FMT_Q8>(a, p.P, p.norm, p.dual, s);
            case FMT_Q4: return pick_aligned_mode<FMT_Q4>(a, p.P, p.norm, p.dual, s);
        }
    }
    switch (job.w.fmt) {
        case FMT_BF16: return pick_mode<FMT_BF16>(a, p.norm, p.dual, s);
        case FMT_Q8: return pick_mode<FMT_Q8>(a, p.norm, p.dual, s);
        case FMT_Q4: return pick_mode<FMT_Q4>(a, p.norm, p.dual, s);
    }
    return fail("HIP backend: unknown weight format.");
}

}  // namespace chip
