// GQA causal attention over the paged KV cache (the math of
// OpsToolbox::attention / attention_head, ops.rs:1357-1467: scores k·q scaled
// by 1/sqrt(head_dim), softmax, weighted value mix), as split-K flash
// decoding:
//
//   attn_kernel: grid (splits, kv_heads, rows); block = 256 threads.
//   Each block owns one KV head, one query row and one contiguous slice of
//   that row's visible positions [0, pos]; it streams the slice in tiles of
//   64 positions (one page-aligned 64 x head_dim tile of K, then of V),
//   scores all G = q_heads / kv_heads query heads of the group against each K
//   row it loads (K and V are read once per group, not once per head), keeps
//   an online softmax (running max / sum) per head and accumulates p * V.
//   With one split it writes the normalised output; otherwise it writes a
//   partial (unnormalised sum, max, denominator) and
//   attn_combine_kernel merges the splits of each (row, q head) in split
//   order, so results are deterministic.
//
// Split boundaries depend only on a row's own context length and the split
// count. Decode is rows == 1; chunked prefill passes the chunk's rows, each
// with its own causal length. The position base comes from a device word in
// the decode graph (pos_dev) or from the host. K/V elements are BF16
// (default) or f32.
#include "kernels.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;
constexpr int TP = 64;  // positions per tile (page_size is a multiple of it)
constexpr int kMaxSplits = 64;

struct AttnArgs {
    const float *q;
    long q_stride;
    const void *k, *v;
    const int32_t *page_table;
    int page_size, kv_heads, q_heads;
    long offset;
    const int32_t *pos_dev;
    float *part;
    float *out;
};

// Eight consecutive K or V elements of one row as f32.
__device__ __forceinline__ void load8(const uint16_t *p, float (&f)[8]) {
    const u32x4 w = *(const u32x4 *)p;
    f[0] = bf16_lo(w[0]); f[1] = bf16_hi(w[0]); f[2] = bf16_lo(w[1]); f[3] = bf16_hi(w[1]);
    f[4] = bf16_lo(w[2]); f[5] = bf16_hi(w[2]); f[6] = bf16_lo(w[3]); f[7] = bf16_hi(w[3]);
}
__device__ __forceinline__ void load8(const float *p, float (&f)[8]) {
    const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
    f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3];
    f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
}

template <int HD, int G, class KT, bool DIRECT>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnArgs a) {
    constexpr int T = HD / 8;          // threads per position row (8 dims each)
    constexpr int P = kThreads / T;    // positions per pass
    constexpr int JW = (G + 3) / 4;    // heads per wave in the softmax step
    __shared__ float s_p[G][TP];
    __shared__ float s_alpha[G];
    __shared__ float s_red[kThreads / 64][G][HD];
    __shared__ float s_l[G];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int d8 = tid % T, pg = tid / T;
    const int split = blockIdx.x, S = gridDim.x;
    const int g = blockIdx.y;
    const int row = blockIdx.z;
    const long pos = (a.pos_dev ? (long)*a.pos_dev : a.offset) + row;
    const long ctx = pos + 1;
    long chunk = (ctx + S - 1) / S;
    chunk = (chunk + TP - 1) / TP * TP;
    const long start = (long)split * chunk;
    const long end = min(start + chunk, ctx);
    const size_t part_head = (size_t)S * (HD + 2);
    float *part = a.part + ((size_t)row * a.q_heads + (size_t)g * G) * part_head + (size_t)split * (HD + 2);

    if (start >= ctx) {  // empty split: contributes nothing to the merge
        if (tid < G) part[tid * part_head + HD] = -INFINITY;
        return;
    }

    const float scale = 1.0f / sqrtf((float)HD);
    float qr[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const float *qp = a.q + (size_t)row * a.q_stride + (size_t)(g * G + j) * HD + d8 * 8;
        const f32x4 q0 = *(const f32x4 *)qp, q1 = *(const f32x4 *)(qp + 4);
        qr[j][0] = q0[0]; qr[j][1] = q0[1]; qr[j][2] = q0[2]; qr[j][3] = q0[3];
        qr[j][4] = q1[0]; qr[j][5] = q1[1]; qr[j][6] = q1[2]; qr[j][7] = q1[3];
    }
    float acc[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    float m_run[JW], l_run[JW];
#pragma unroll
    for (int i = 0; i < JW; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
    }

    for (long t0 = start; t0 < end; t0 += TP) {
        const int page = a.page_table[t0 / a.page_size];
        const long slot0 = t0 % a.page_size;
        const size_t tile_off = (((size_t)page * a.kv_heads + g) * a.page_size + slot0) * HD;
        const KT *kt = (const KT *)a.k + tile_off;
        const KT *vt = (const KT *)a.v + tile_off;
        // V rows are independent of the scores: start their loads now.
        float vf[TP / P][8];
#pragma unroll
        for (int p = 0; p < TP / P; ++p) {
            const int pi = p * P + pg;
            if (t0 + pi < end) load8(vt + (size_t)pi * HD + d8 * 8, vf[p]);
        }
        // Scores of every head of the group for the tile's rows.
#pragma unroll
        for (int p = 0; p < TP / P; ++p) {
            const int pi = p * P + pg;
            const bool valid = t0 + pi < end;
            float dot[G];
#pragma unroll
            for (int j = 0; j < G; ++j) dot[j] = 0.f;
            if (valid) {
                float kf[8];
                load8(kt + (size_t)pi * HD + d8 * 8, kf);
#pragma unroll
                for (int j = 0; j < G; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e) dot[j] = fmaf(kf[e], qr[j][e], dot[j]);
            }
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float sum = group_sum<T>(dot[j]);
                if (d8 == 0) s_p[j][pi] = valid ? sum * scale : -INFINITY;
            }
        }
        __syncthreads();
        // Online softmax per head: one wave per head, one lane per position.
#pragma unroll
        for (int i = 0; i < JW; ++i) {
            const int j = wave + 4 * i;
            if (j < G) {
                const float sc = s_p[j][lane];
                const float m_new = fmaxf(m_run[i], wave_max(sc));
                const float pv = sc == -INFINITY ? 0.f : expf(sc - m_new);
                s_p[j][lane] = pv;
                const float l_tile = wave_sum(pv);
                const float alpha = m_run[i] == -INFINITY ? 0.f : expf(m_run[i] - m_new);
                l_run[i] = l_run[i] * alpha + l_tile;
                m_run[i] = m_new;
                if (lane == 0) s_alpha[j] = alpha;
            }
        }
        __syncthreads();
        // acc = acc * alpha + sum_p p * V[p].
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float al = s_alpha[j];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[j][e] *= al;
        }
#pragma unroll
        for (int p = 0; p < TP / P; ++p) {
            const int pi = p * P + pg;
            if (t0 + pi < end) {
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const float pj = s_p[j][pi];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(pj, vf[p][e], acc[j][e]);
                }
            }
        }
        __syncthreads();
    }
    // Reduce acc over the position groups: lanes d8, d8+T, ... of a wave,
    // then across the 4 waves through LDS.
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[j][e];
#pragma unroll
            for (int off = T; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
            acc[j][e] = v;
        }
    if (lane < T) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) s_red[wave][j][d8 * 8 + e] = acc[j][e];
    }
#pragma unroll
    for (int i = 0; i < JW; ++i) {
        const int j = wave + 4 * i;
        if (j < G && lane == 0) {
            if constexpr (DIRECT) {
                s_l[j] = l_run[i];
            } else {
                part[j * part_head + HD] = m_run[i];
                part[j * part_head + HD + 1] = l_run[i];
            }
        }
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += kThreads) {
        const int j = t / HD, d = t % HD;
        const float o = s_red[0][j][d] + s_red[1][j][d] + s_red[2][j][d] + s_red[3][j][d];
        if constexpr (DIRECT) a.out[((size_t)row * a.q_heads + g * G + j) * HD + d] = o / s_l[j];
        else part[j * part_head + d] = o;
    }
}

// Merge the splits of one (row, q head) in split order: one wave turns the
// split maxima into weights w_s = exp(m_s - M) and 1 / sum_s w_s l_s, then
// all threads sum w_s * o_s[d] over the non-empty splits.
template <int HD>
__global__ __launch_bounds__(kThreads) void attn_combine_kernel(const float *part, int S, int q_heads, float *out) {
    constexpr int GR = kThreads / HD;  // split groups
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_inv;
    __shared__ float s_o[GR][HD];
    const int h = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const float *p = part + ((size_t)row * q_heads + h) * (size_t)S * (HD + 2);
    if (tid < 64) {
        const float m = tid < S ? p[(size_t)tid * (HD + 2) + HD] : -INFINITY;
        const float M = wave_max(m);
        const float w = m == -INFINITY ? 0.f : expf(m - M);
        const float l = w != 0.f ? p[(size_t)tid * (HD + 2) + HD + 1] : 0.f;
        const float L = wave_sum(w * l);
        if (tid < S) s_w[tid] = w;
        if (tid == 0) s_inv = 1.0f / L;
    }
    __syncthreads();
    const int d = tid % HD, grp = tid / HD;
    float o = 0.f;
    for (int s = grp; s < S; s += GR) {
        const float w = s_w[s];
        if (w != 0.f) o = fmaf(w, p[(size_t)s * (HD + 2) + d], o);
    }
    s_o[grp][d] = o;
    __syncthreads();
    if (tid < HD) {
        float sum = s_o[0][tid];
#pragma unroll
        for (int k = 1; k < GR; ++k) sum += s_o[k][tid];
        out[((size_t)row * q_heads + h) * HD + tid] = sum * s_inv;
    }
}

template <int HD, int G, class KT>
int launch_hgk(const AttnJob &j, const AttnArgs &a, hipStream_t s) {
    const dim3 grid(j.splits, j.g.kv_heads, j.rows);
    if (j.splits == 1) {
        hipLaunchKernelGGL((attn_kernel<HD, G, KT, true>), grid, dim3(kThreads), 0, s, a);
        CHIP_CHECK(hipGetLastError());
        return 0;
    }
    hipLaunchKernelGGL((attn_kernel<HD, G, KT, false>), grid, dim3(kThreads), 0, s, a);
    CHIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(j.q_heads, j.rows), dim3(kThreads), 0, s, a.part, j.splits,
                       j.q_heads, a.out);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

template <int HD, int G>
int launch_hg(const AttnJob &j, const AttnArgs &a, hipStream_t s) {
    if (j.g.kv_f32) return launch_hgk<HD, G, float>(j, a, s);
    return launch_hgk<HD, G, uint16_t>(j, a, s);
}

template <int HD>
int launch_h(const AttnJob &j, const AttnArgs &a, int G, hipStream_t s) {
    switch (G) {
        case 1: return launch_hg<HD, 1>(j, a, s);
        case 2: return launch_hg<HD, 2>(j, a, s);
        case 3: return launch_hg<HD, 3>(j, a, s);
        case 4: return launch_hg<HD, 4>(j, a, s);
        case 5: return launch_hg<HD, 5>(j, a, s);
        case 6: return launch_hg<HD, 6>(j, a, s);
        case 7: return launch_hg<HD, 7>(j, a, s);
        case 8: return launch_hg<HD, 8>(j, a, s);
    }
    return fail("HIP backend: attention supports 1..8 query heads per KV head.");
}

}  // namespace

size_t attention_part_floats(size_t rows, int q_heads, int splits, int head_dim) {
    return rows * (size_t)q_heads * (size_t)splits * (size_t)(head_dim + 2);
}

int attention_max_splits() { return kMaxSplits; }

int launch_attention(const AttnJob &j, hipStream_t s) {
    if (j.rows == 0) return 0;
    if (!j.q || !j.out || !j.k || !j.v || !j.g.page_table || (j.splits > 1 && !j.part))
        return fail("HIP backend: attention is missing a buffer.");
    if (j.g.kv_heads <= 0 || j.q_heads <= 0 || j.q_heads % j.g.kv_heads)
        return fail("HIP backend: q_heads must be a multiple of kv_heads.");
    if (j.g.page_size <= 0 || j.g.page_size % TP)
        return fail("HIP backend: the KV page size must be a multiple of 64 positions.");
    if (j.splits <= 0 || j.splits > kMaxSplits || j.rows > 65535 || j.q_heads > 65535)
        return fail("HIP backend: attention grid out of range.");
    AttnArgs a{};
    a.q = j.q;
    a.q_stride = (long)j.q_stride;
    a.k = j.k;
    a.v = j.v;
    a.page_table = j.g.page_table;
    a.page_size = j.g.page_size;
    a.kv_heads = j.g.kv_heads;
    a.q_heads = j.q_heads;
    a.offset = (long)j.offset;
    a.pos_dev = j.pos_dev;
    a.part = j.part;
    a.out = j.out;
    const int G = j.q_heads / j.g.kv_heads;
    if (j.g.head_dim == 64) return launch_h<64>(j, a, G, s);
    if (j.g.head_dim == 128) return launch_h<128>(j, a, G, s);
    return fail("HIP backend: attention supports head_dim 64 and 128.");
}

}  // namespace chip
