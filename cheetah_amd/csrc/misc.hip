// Small per-row kernels of the decoder forward: embedding gather, RMSNorm
// rows, fused RoPE + paged BF16 KV append, and greedy argmax.
#include "kernels.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;

// embedding_row_into (ops.rs:1083-1099): BF16 -> f32 widening. blockIdx.y
// is the row; each thread widens up to 8 consecutive elements of one block
// of 8 * kThreads, with one 16-byte load when the row allows it.
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t *__restrict__ table, int hidden,
                                                         const uint32_t *__restrict__ tokens, float *__restrict__ out) {
    const uint32_t tok = tokens[blockIdx.y];
    const uint16_t *src = table + (size_t)tok * hidden;
    float *dst = out + (size_t)blockIdx.y * hidden;
    const int i0 = (blockIdx.x * kThreads + threadIdx.x) * 8;
    if (i0 >= hidden) return;
    if (i0 + 8 <= hidden && hidden % 8 == 0 && ((uintptr_t)table & 15) == 0 && ((uintptr_t)out & 15) == 0) {
        const u32x4 w = *(const u32x4 *)(src + i0);
        *(f32x4 *)(dst + i0) = f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
        *(f32x4 *)(dst + i0 + 4) = f32x4{bf16_lo(w[2]), bf16_hi(w[2]), bf16_lo(w[3]), bf16_hi(w[3])};
    } else {
        for (int i = i0; i < min(i0 + 8, hidden); ++i) dst[i] = bf16_f32(src[i]);
    }
}

// rmsnorm (ops.rs:646-652): x * (inv * gain), inv = 1 / sqrt(mean(x^2) + eps).
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const float *x, const uint16_t *gain, float eps, int n,
                                                                float *out, uint16_t *xh, uint16_t *xl) {
    __shared__ float red[kThreads / 64];
    const float *src = x + (size_t)blockIdx.x * n;
    float *dst = out + (size_t)blockIdx.x * n;
    // Eight of the thread's elements loaded at a time; squares summed in
    // element order.
    float ss = 0.f;
    for (int base = threadIdx.x; base < n; base += 8 * kThreads) {
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = base + kThreads * k;
            t[k] = i < n ? src[i] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (base + kThreads * k < n) ss = fmaf(t[k], t[k], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(total / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = src[i] * (inv * bf16_f32(gain[i]));
        dst[i] = v;
        if (xh) {
            const size_t o = (size_t)blockIdx.x * n + i;
            const __bf16 hb = (__bf16)v;
            xh[o] = __builtin_bit_cast(uint16_t, hb);
            xl[o] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)hb));
        }
    }
}

// A residual GEMM's split-K reduction (its nchunks stored sums folded in a
// single matrix's association: the first ceil(n / 2) left to right, the
// rest left to right, then the two added; then the epilogue of
// gemm_reduce_kernel: row scale, bias, residual add) fused with the row
// RMSNorm that follows it; the norm's sum of squares runs over the same
// per-thread order as rmsnorm_rows_kernel, so every output has the bits of
// the two separate kernels.
__global__ __launch_bounds__(kThreads) void residual_rmsnorm_rows_kernel(const float *ws, int nchunks, const float *sc,
                                                                         const float *bias, float *hidden, int rows,
                                                                         int n, const uint16_t *gain, float eps,
                                                                         float *out, uint16_t *xh, uint16_t *xl) {
    __shared__ float red[kThreads / 64];
    const int m = blockIdx.x;
    const size_t MN = (size_t)rows * n;
    float *h = hidden + (size_t)m * n;
    // A thread's elements i = tid + kThreads k, EPT of them per pass: their
    // residuals and eight chunk sums each are loaded together (one memory
    // round trip per eight chunks, not per element), then each element folds
    // its chunks (two halves, each in chunk order) and the squares are summed
    // in element order.
    constexpr int EPT = 4, ZB = 8;
    const int hs = (nchunks + 1) / 2;  // sums in the first half
    float ss = 0.f;
    for (int base = 0; base < n; base += EPT * kThreads) {
        float v[EPT], v2[EPT], hv[EPT];
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int i = base + (int)threadIdx.x + kThreads * k;
            v[k] = v2[k] = 0.f;
            hv[k] = i < n ? h[i] : 0.f;
        }
        for (int z0 = 0; z0 < nchunks; z0 += ZB) {
            float t[ZB][EPT];
#pragma unroll
            for (int j = 0; j < ZB; ++j)
#pragma unroll
                for (int k = 0; k < EPT; ++k) {
                    const int i = base + (int)threadIdx.x + kThreads * k;
                    t[j][k] = z0 + j < nchunks && i < n ? ws[(size_t)(z0 + j) * MN + (size_t)m * n + i] : 0.f;
                }
#pragma unroll
            for (int j = 0; j < ZB; ++j)
#pragma unroll
                for (int k = 0; k < EPT; ++k) {
                    if (z0 + j < hs) v[k] += t[j][k];
                    else if (z0 + j < nchunks) v2[k] += t[j][k];
                }
        }
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int i = base + (int)threadIdx.x + kThreads * k;
            if (i < n) {
                float x = hs < nchunks ? v[k] + v2[k] : v[k];
                if (sc) x = x * sc[i];
                if (bias) x = x + bias[i];
                const float r = hv[k] + x;
                h[i] = r;
                ss = fmaf(r, r, ss);
            }
        }
    }
    if (!gain) return;
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(total / (float)n + eps);
    float *dst = out + (size_t)m * n;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const float v = h[i] * (inv * bf16_f32(gain[i]));
        dst[i] = v;
        if (xh) {
            const size_t o = (size_t)m * n + i;
            const __bf16 hb = (__bf16)v;
            xh[o] = __builtin_bit_cast(uint16_t, hb);
            xl[o] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)hb));
        }
    }
}

// residual_rmsnorm_rows_kernel for a row that fits the block's registers
// (n <= EPT * kThreads) with at most ZM stored sums: every residual, stored
// sum, scale, bias and gain of the thread's elements is loaded in one round
// trip, and the row stays in registers for the norm instead of being read
// back. The arithmetic and its order are residual_rmsnorm_rows_kernel's
// (the same bits).
template <int EPT, int ZM>
__global__ __launch_bounds__(kThreads) void residual_rmsnorm_rows_reg_kernel(const float *ws, int nchunks,
                                                                             const float *sc, const float *bias,
                                                                             float *hidden, int rows, int n,
                                                                             const uint16_t *gain, float eps,
                                                                             float *out, uint16_t *xh, uint16_t *xl) {
    __shared__ float red[kThreads / 64];
    const int m = blockIdx.x;
    const size_t MN = (size_t)rows * n;
    float *h = hidden + (size_t)m * n;
    const int hs = (nchunks + 1) / 2;  // sums in the first half
    float hv[EPT], scv[EPT], bv[EPT], gv[EPT], t[ZM][EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int i = (int)threadIdx.x + kThreads * k;
        const bool in = i < n;
        hv[k] = in ? h[i] : 0.f;
        scv[k] = sc && in ? sc[i] : 0.f;
        bv[k] = bias && in ? bias[i] : 0.f;
        gv[k] = gain && in ? bf16_f32(gain[i]) : 0.f;
#pragma unroll
        for (int j = 0; j < ZM; ++j) t[j][k] = j < nchunks && in ? ws[(size_t)j * MN + (size_t)m * n + i] : 0.f;
    }
    float r[EPT], ss = 0.f;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int i = (int)threadIdx.x + kThreads * k;
        r[k] = 0.f;
        if (i < n) {
            float v = 0.f, v2 = 0.f;
#pragma unroll
            for (int j = 0; j < ZM; ++j) {
                if (j < hs) v += t[j][k];
                else if (j < nchunks) v2 += t[j][k];
            }
            float x = hs < nchunks ? v + v2 : v;
            if (sc) x = x * scv[k];
            if (bias) x = x + bv[k];
            r[k] = hv[k] + x;
            h[i] = r[k];
            ss = fmaf(r[k], r[k], ss);
        }
    }
    if (!gain) return;
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(total / (float)n + eps);
    float *dst = out + (size_t)m * n;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int i = (int)threadIdx.x + kThreads * k;
        if (i < n) {
            const float v = r[k] * (inv * gv[k]);
            dst[i] = v;
            if (xh) {
                const size_t o = (size_t)m * n + i;
                const __bf16 hb = (__bf16)v;
                xh[o] = __builtin_bit_cast(uint16_t, hb);
                xl[o] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)hb));
            }
        }
    }
}

// rope_heads (ops.rs:693-740) with the angle's cos/sin read from a table the
// host filled with the same libm powf/sinf/cosf the reference calls, so q and
// k come out bit-identical to the CPU path for identical inputs; then
// cache_append (ops.rs:1329-1332) into the paged BF16 cache.
__device__ __forceinline__ void store_kv(uint16_t *p, float v) { *p = f32_bf16_rne(v); }
__device__ __forceinline__ void store_kv(float *p, float v) { *p = v; }


// One thread per output element: blockIdx.y is the row, blockIdx.x a run of
// kThreads elements over [q | k] (each k element also appends its v). A
// thread issues its few loads at once, so a row costs one memory round trip
// whatever its width.
template <class KT, bool SUM>
__global__ __launch_bounds__(kThreads) void rope_append_kernel(const float *__restrict__ qkv, float *__restrict__ qrot,
                                                               int q_heads, int kv_heads, int head_dim, int rotary_dim,
                                                               const float *__restrict__ cos_t,
                                                               const float *__restrict__ sin_t,
                                                               const int32_t *__restrict__ page_table, int page_size,
                                                               KT *__restrict__ kc, KT *__restrict__ vc, long offset,
                                                               const int32_t *__restrict__ pos_dev,
                                                               const float *__restrict__ ws, int nchunks,
                                                               const float *__restrict__ sc,
                                                               const float *__restrict__ bias) {
    const int row = blockIdx.y, rows = gridDim.y;
    const int t = blockIdx.x * kThreads + threadIdx.x;
    const int q_dim = q_heads * head_dim, kv_dim = kv_heads * head_dim, width = q_dim + 2 * kv_dim;
    if (t >= q_dim + kv_dim) return;
    const long pos = (pos_dev ? (long)*pos_dev : offset) + row;
    const float *q = qkv + (size_t)row * width;
    // Element col of this row: stored, or (SUM) the deferred GEMM's stored
    // sums folded in its association (the first ceil(n / 2) left to right,
    // the rest left to right, the two added), then scale and bias (its
    // epilogue, same bits).
    auto val = [&](int col) -> float {
        if constexpr (SUM) {
            const int hs = (nchunks + 1) / 2;
            float v = 0.f, v2 = 0.f;
            for (int z = 0; z < hs; ++z) v += ws[((size_t)z * rows + row) * width + col];
            for (int z = hs; z < nchunks; ++z) v2 += ws[((size_t)z * rows + row) * width + col];
            if (hs < nchunks) v = v + v2;
            if (sc) v = v * sc[col];
            if (bias) v = v + bias[col];
            return v;
        } else {
            return q[col];
        }
    };
    const int half = rotary_dim / 2;
    const float *cr = cos_t + (size_t)pos * half;
    const float *sr = sin_t + (size_t)pos * half;
    // rope_elem's arithmetic on element d of the head starting at column base.
    auto rot = [&](int base, int d) -> float {
        if (d >= rotary_dim) return val(base + d);
        const int i = d < half ? d : d - half;
        const float a = val(base + 2 * i), b = val(base + 2 * i + 1), c = cr[i], s = sr[i];
        return d < half ? a * c - b * s : b * c + a * s;
    };
    if (t < q_dim) {
        const int h = t / head_dim, d = t % head_dim;
        qrot[(size_t)row * q_dim + t] = rot(h * head_dim, d);
        return;
    }
    const int u = t - q_dim;
    const int h = u / head_dim, d = u % head_dim;
    const int page = page_table[pos / page_size];
    const int slot = (int)(pos % page_size);
    const float kv = rot(q_dim + h * head_dim, d);
    const size_t off = (((size_t)page * kv_heads + h) * page_size + slot) * head_dim + d;
    store_kv(kc + off, kv);
    store_kv(vc + off, val(q_dim + kv_dim + u));
}

__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const uint8_t *src, uint8_t *dst, const int32_t *map,
                                                               size_t row_bytes) {
    const uint8_t *s = src + (size_t)map[blockIdx.x] * row_bytes;
    uint8_t *d = dst + (size_t)blockIdx.x * row_bytes;
    for (size_t i = threadIdx.x; i < row_bytes; i += kThreads) d[i] = s[i];
}

// Total order of f32::total_cmp as a signed integer key.
__device__ __forceinline__ int total_key(float f) {
    int i = __float_as_int(f);
    return i ^ (int)(((unsigned)(i >> 31)) >> 1);
}

// max_by(total_cmp) keeps the LAST maximal element (engine.rs:2247-2253):
// among equal keys the larger index wins.
__device__ __forceinline__ void better(int &key, uint32_t &idx, int k2, uint32_t i2) {
    if (k2 > key || (k2 == key && i2 > idx)) {
        key = k2;
        idx = i2;
    }
}

__device__ __forceinline__ void block_argmax(int &key, uint32_t &idx) {
    __shared__ int skey[kThreads / 64];
    __shared__ uint32_t sidx[kThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        int k2 = __shfl_xor(key, off, 64);
        uint32_t i2 = __shfl_xor(idx, off, 64);
        better(key, idx, k2, i2);
    }
    if ((threadIdx.x & 63) == 0) {
        skey[threadIdx.x >> 6] = key;
        sidx[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    key = skey[0];
    idx = sidx[0];
    for (int w = 1; w < kThreads / 64; ++w) better(key, idx, skey[w], sidx[w]);
}

constexpr int kArgmaxBlocks = 64;

__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float *x, int n, int *pkey, uint32_t *pidx) {
    int key = INT_MIN;
    uint32_t idx = 0;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
        better(key, idx, total_key(x[i]), (uint32_t)i);
    block_argmax(key, idx);
    if (threadIdx.x == 0) {
        pkey[blockIdx.x] = key;
        pidx[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(kThreads) void argmax_final_kernel(const int *pkey, const uint32_t *pidx, int parts,
                                                                uint32_t *out, int32_t *step, uint32_t *hist,
                                                                long hist_cap) {
    int key = INT_MIN;
    uint32_t idx = 0;
    for (int i = threadIdx.x; i < parts; i += kThreads) better(key, idx, pkey[i], pidx[i]);
    block_argmax(key, idx);
    if (threadIdx.x == 0) {
        if (out) *out = idx;
        if (step) {
            const long next = (long)step[1] + 1;
            if (hist && next < hist_cap) hist[next] = idx;
            step[0] = (int32_t)idx;
            step[1] = (int32_t)next;
        }
    }
}

}  // namespace

int launch_embed(const uint16_t *table, size_t hidden, const uint32_t *tokens, size_t rows, float *out,
                 hipStream_t s) {
    if (rows == 0) return 0;
    if (rows > 65535) return fail("HIP backend: embedding takes at most 65535 rows per launch.");
    const dim3 grid((unsigned)((hidden + 8 * kThreads - 1) / (8 * kThreads)), (unsigned)rows);
    hipLaunchKernelGGL(embed_kernel, grid, dim3(kThreads), 0, s, table, (int)hidden, tokens, out);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int launch_rmsnorm_rows(const float *x, const uint16_t *gain, float eps, size_t rows, size_t n, float *out,
                        hipStream_t s, uint16_t *xh, uint16_t *xl) {
    if (rows == 0) return 0;
    if (!xh != !xl) return fail("HIP backend: rmsnorm needs both BF16 halves or neither.");
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(kThreads), 0, s, x, gain, eps, (int)n, out, xh, xl);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int launch_residual_rmsnorm_rows(const float *ws, int nchunks, const float *sc, const float *bias, float *hidden,
                                 size_t rows, size_t n, const uint16_t *gain, float eps, float *out, hipStream_t s,
                                 uint16_t *xh, uint16_t *xl) {
    if (rows == 0) return 0;
    if (!ws || nchunks <= 0 || !hidden || (gain && !out)) return fail("HIP backend: residual norm is missing a buffer.");
    if (!xh != !xl) return fail("HIP backend: rmsnorm needs both BF16 halves or neither.");
    if (rows > (size_t)INT32_MAX || n > (size_t)INT32_MAX) return fail("HIP backend: residual norm shape too large.");
    // A row of 1,025 to 4,096 with at most four stored sums (a GEMM's two halves) in registers: one load round
    // trip instead of one per 1,024 elements, and no read-back for the norm. Measured: Llama-3-8B Q4 512-row
    // chunks 26 -> 18 us per call, prefill 20.4K -> 20.7K tok/s; the same form for Qwen2-0.5B's 896-wide rows
    // (one pass either way) was slower (prefill 63.2K -> 60.1K).
    if (n > 4 * kThreads && n <= 16 * kThreads && nchunks <= 4)
        hipLaunchKernelGGL((residual_rmsnorm_rows_reg_kernel<16, 4>), dim3((unsigned)rows), dim3(kThreads), 0, s, ws,
                           nchunks, sc, bias, hidden, (int)rows, (int)n, gain, eps, out, xh, xl);
    else
        hipLaunchKernelGGL(residual_rmsnorm_rows_kernel, dim3((unsigned)rows), dim3(kThreads), 0, s, ws, nchunks, sc,
                           bias, hidden, (int)rows, (int)n, gain, eps, out, xh, xl);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int qkv_perm_row(int stored, int q_heads, int kv_heads, int head_dim, int rotary_dim) {
    const int q_dim = q_heads * head_dim, k_end = q_dim + kv_heads * head_dim;
    if (stored >= k_end) return stored;  // v rows
    const int head_base = stored - stored % head_dim, d = stored % head_dim;
    if (d >= rotary_dim) return stored;
    const int half = rotary_dim / 2;
    return head_base + (d % 2 == 0 ? d / 2 : half + d / 2);
}

int launch_rope_append(const float *qkv, float *qrot, size_t rows, int q_heads, const KvGeom &g, const KvLayer &kv,
                       const float *rope_cos, const float *rope_sin, int rotary_dim, size_t offset,
                       const int32_t *pos_dev, hipStream_t s, const float *ws, int nchunks, const float *sc,
                       const float *bias) {
    if (rows == 0) return 0;
    if (rotary_dim <= 0 || rotary_dim > g.head_dim || rotary_dim % 2)
        return fail("HIP backend: rotary_dim must be even and at most head_dim.");
    const int width = q_heads * g.head_dim + g.kv_heads * g.head_dim;
    const dim3 grid((width + kThreads - 1) / kThreads, (unsigned)rows);
    if (rows > 65535) return fail("HIP backend: rope_append takes at most 65535 rows per launch.");
    if (nchunks > 0 && !ws) return fail("HIP backend: rope_append's deferred sums have no workspace.");
#define CHIP_ROPE(KT, SUM)                                                                                      \
    hipLaunchKernelGGL((rope_append_kernel<KT, SUM>), grid, dim3(kThreads), 0, s, qkv, qrot, q_heads, g.kv_heads, \
                       g.head_dim, rotary_dim, rope_cos, rope_sin, g.page_table, g.page_size, (KT *)kv.k,         \
                       (KT *)kv.v, (long)offset, pos_dev, ws, nchunks, sc, bias)
    if (g.kv_f32) {
        if (nchunks > 0) CHIP_ROPE(float, true);
        else CHIP_ROPE(float, false);
    } else {
        if (nchunks > 0) CHIP_ROPE(uint16_t, true);
        else CHIP_ROPE(uint16_t, false);
    }
#undef CHIP_ROPE
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int launch_gather_rows(const uint8_t *src, uint8_t *dst, const int32_t *map, size_t rows, size_t row_bytes,
                       hipStream_t s) {
    if (rows == 0) return 0;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(rows), dim3(kThreads), 0, s, src, dst, map, row_bytes);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

size_t argmax_scratch_bytes() { return kArgmaxBlocks * (sizeof(int) + sizeof(uint32_t)); }

int launch_argmax(const float *logits, size_t n, uint32_t *out_token, int32_t *step, uint32_t *hist,
                  size_t hist_cap, void *scratch, hipStream_t s) {
    if (n == 0 || n > (size_t)INT32_MAX) return fail("HIP backend: argmax over an empty or oversized vector.");
    int *pkey = (int *)scratch;
    uint32_t *pidx = (uint32_t *)(pkey + kArgmaxBlocks);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxBlocks), dim3(kThreads), 0, s, logits, (int)n, pkey, pidx);
    CHIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kThreads), 0, s, (const int *)pkey, (const uint32_t *)pidx,
                       kArgmaxBlocks, out_token, step, hist, (long)hist_cap);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

}  // namespace chip
