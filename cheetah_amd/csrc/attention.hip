// GQA causal attention over the paged KV cache (the math of
// OpsToolbox::attention / attention_head, ops.rs:1357-1467: scores k·q scaled
// by 1/sqrt(head_dim), softmax, weighted value mix), as split-K flash
// decoding:
//
//   attn_kernel (f32 K/V; BF16 K/V decode runs on the matrix cores,
//   attn_dec_mfma_kernel below): grid (splits, kv_heads, rows); block = 256
//   threads.
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
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "kernels.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;
constexpr int TP = 64;  // positions per tile (page_size is a multiple of it)
constexpr int kMaxSplits = 128;

// Block barrier that waits on LDS traffic only (outstanding global loads
// stay in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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
    // Fused decode RoPE (attn_dec_mfma_kernel<.., ROPE>): raw QKV row and
    // the cos/sin table; K/V are then also written (the new row).
    const float *qkv;
    const float *rope_cos, *rope_sin;
    int rotary_dim;
    // Chunked prefill: BF16 halves of out (null: not written).
    uint16_t *out_hi, *out_lo;
};

// hi = bf16(v), lo = bf16(v - hi) (hardware round-to-nearest-even) of four
// consecutive outputs at element i: the split the next GEMM takes as input.
__device__ __forceinline__ void store_halves4(uint16_t *hi, uint16_t *lo, size_t i, f32x4 v) {
    uint16_t h[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const __bf16 hb = (__bf16)v[q];
        h[q] = __builtin_bit_cast(uint16_t, hb);
        l[q] = __builtin_bit_cast(uint16_t, (__bf16)(v[q] - (float)hb));
    }
    *(uint2 *)(hi + i) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    *(uint2 *)(lo + i) = make_uint2((uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16));
}

// Eight consecutive K or V elements as loaded (converted to f32 at use), so
// a whole tile can be in flight while the previous one computes.
template <class KT>
struct Raw8;
template <>
struct Raw8<uint16_t> {
    u32x4 w;
    __device__ void load(const uint16_t *p) { w = *(const u32x4 *)p; }
    __device__ void get(float (&f)[8]) const {
        f[0] = bf16_lo(w[0]); f[1] = bf16_hi(w[0]); f[2] = bf16_lo(w[1]); f[3] = bf16_hi(w[1]);
        f[4] = bf16_lo(w[2]); f[5] = bf16_hi(w[2]); f[6] = bf16_lo(w[3]); f[7] = bf16_hi(w[3]);
    }
};
template <>
struct Raw8<float> {
    f32x4 a, b;
    __device__ void load(const float *p) {
        a = *(const f32x4 *)p;
        b = *(const f32x4 *)(p + 4);
    }
    __device__ void get(float (&f)[8]) const {
        f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3];
        f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
    }
};

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

    // K/V tiles ping-pong between two register sets: tile t0 + TP loads while
    // tile t0 computes. A position past `end` reads the row at end - 1 (the
    // compute masks it), and the tile barriers wait on LDS only, so the loads
    // of the next tile stay in flight across the current tile's barriers.
    // (Four sets, three tiles in flight, measured slower: 254 registers.)
    constexpr int NB = 2;
    Raw8<KT> bk[NB][TP / P], bv[NB][TP / P];
    const long last_tile = start + (end - 1 - start) / TP * TP;
    auto issue = [&](long t, Raw8<KT> (&kr)[TP / P], Raw8<KT> (&vr)[TP / P]) {
        t = min(t, last_tile);
        const int page = a.page_table[t / a.page_size];
        const size_t tile_off = (((size_t)page * a.kv_heads + g) * a.page_size + t % a.page_size) * HD;
        const KT *kt = (const KT *)a.k + tile_off;
        const KT *vt = (const KT *)a.v + tile_off;
        const int rmax = (int)(end - 1 - t);
#pragma unroll
        for (int p = 0; p < TP / P; ++p) {
            const int r = min(p * P + pg, rmax);
            kr[p].load(kt + (size_t)r * HD + d8 * 8);
            vr[p].load(vt + (size_t)r * HD + d8 * 8);
        }
    };
    auto tile = [&](long t0, const Raw8<KT> (&kc)[TP / P], const Raw8<KT> (&vc)[TP / P]) {
        // Scores of every head of the group for the tile's rows (each K row
        // widened to f32 where it is used).
#pragma unroll
        for (int p = 0; p < TP / P; ++p) {
            const int pi = p * P + pg;
            const bool valid = t0 + pi < end;
            float kf[8];
            kc[p].get(kf);
            float dot[G];
#pragma unroll
            for (int j = 0; j < G; ++j) dot[j] = 0.f;
            if (valid) {
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
        lds_barrier();
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
        lds_barrier();
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
                float vf[8];
                vc[p].get(vf);
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const float pj = s_p[j][pi];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(pj, vf[e], acc[j][e]);
                }
            }
        }
        lds_barrier();
    };
    issue(start, bk[0], bv[0]);
    if (end - start <= TP) {
        tile(start, bk[0], bv[0]);
    } else {
#pragma unroll
        for (int b = 1; b < NB; ++b) issue(start + b * TP, bk[b], bv[b]);
        for (long t0 = start; t0 < end; t0 += NB * TP) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const long tb = t0 + b * TP;
                if (b == 0 || tb < end) tile(tb, bk[b], bv[b]);
                issue(tb + NB * TP, bk[b], bv[b]);
            }
        }
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

// ---------------------------------------------------------------------------
// Decode attention on the matrix cores (BF16 KV, head_dim 64 or 128, up to 8
// query heads per KV head): grid (splits, kv_heads, rows) as attn_kernel, the
// same split boundaries and partial layout. The block's positions are cut
// into 32-position tiles dealt round-robin to its 4 waves; each wave runs its
// own online softmax over its tiles with no block barrier, and the 4 wave
// partials are merged in wave order at the end.
//
// Per tile, with v_mfma_f32_16x16x32_bf16 (lane L: n = L % 16, kg = L / 16):
//   S^T = K Q^T  A = K rows straight from global memory: M-block mb's row m
//                is position t + 8(m/4) + 4mb + m%4; B = the group's queries
//                as hi/lo BF16 halves of the f32 values (heads >= G zero).
//                Lane L then holds the scores of head n at positions
//                t + 8kg + 4mb + j, j = 0..3.
//   O^T += V^T P^T  B = those 8 probabilities (hi/lo halves) exactly as they
//                sit in the lane; A = V^T read from a per-wave LDS copy of the
//                V tile with ds_read_b64_tr_b16 (lane L gets V[t + 8kg + e]
//                [16db + n], e = 0..7, in two reads of four).
// The V tile is stored row-major with the 16-byte chunks of row r permuted
// (chunk c at slot c ^ vswz(r)) so the transposing reads of a half wave hit
// distinct banks. Every K/V load is issued unconditionally (positions past
// the end re-read the last one and are masked), so tile i + 1 streams in
// while tile i computes.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <int HD>
__device__ __forceinline__ int vswz(int r) {
    if constexpr (HD == 128) return 2 * ((r & 3) | ((r >> 1) & 4));
    else return 2 * (((r >> 1) & 1) | ((r >> 2) & 2));
}

__device__ __forceinline__ void split_hilo(const float (&v)[8], bf16x8_t &hi, bf16x8_t &lo) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        hi[q] = (__bf16)v[q];
        lo[q] = (__bf16)(v[q] - (float)hi[q]);
    }
}

template <int HD, int G, bool DIRECT, bool ROPE>
__global__ __launch_bounds__(kThreads) void attn_dec_mfma_kernel(AttnArgs a) {
    constexpr int TW = 32;             // positions per wave tile
    constexpr int NS = HD / 32;        // K steps of the score product
    constexpr int NDB = HD / 16;       // 16-dim blocks of the value product
    constexpr int CH = HD / 8;         // 16-byte chunks per K/V row
    constexpr int VI = TW * CH / 64;   // V loads per lane per tile
    constexpr int ROWB = HD * 2;       // bytes per K/V row
    __shared__ __attribute__((aligned(16))) uint8_t s_v[4][TW * ROWB];
    __shared__ float s_o[4][G][HD];
    __shared__ float s_m[4][G], s_l[4][G];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int n = lane & 15, kg = lane >> 4;
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
        if (threadIdx.x < G) part[threadIdx.x * part_head + HD] = -INFINITY;
        return;
    }

    // ROPE: the block whose range ends at the context holds position pos,
    // whose K/V row is not in the cache yet. The wave whose tile holds it
    // rotates k (rope_elem, as launch_rope_append), rounds K and V to BF16,
    // appends them to the cache and keeps them in LDS to patch into its
    // tile registers (bits equal to what the cache will hold).
    __shared__ __attribute__((aligned(16))) uint16_t s_new[2][HD];
    const int q_dim = a.q_heads * HD, kv_dim = a.kv_heads * HD, half = a.rotary_dim / 2;
    const float *qkv_row = ROPE ? a.qkv + (size_t)row * (q_dim + 2 * kv_dim) : nullptr;
    const float *cr = ROPE ? a.rope_cos + (size_t)pos * half : nullptr;
    const float *sr = ROPE ? a.rope_sin + (size_t)pos * half : nullptr;
    const int pos_tile = (int)((pos - start) / TW);  // tile index of pos in this block's range
    const bool has_new = ROPE && end == ctx;
    if constexpr (ROPE) {
        if (has_new && wave == pos_tile % 4) {
            const float *kr = qkv_row + q_dim + g * HD, *vr = qkv_row + q_dim + kv_dim + g * HD;
            const int page = a.page_table[pos / a.page_size];
            const size_t off = (((size_t)page * a.kv_heads + g) * a.page_size + pos % a.page_size) * HD;
#pragma unroll
            for (int d = lane; d < HD; d += 64) {
                const uint16_t kb = f32_bf16_rne(rope_elem(kr, d, half, a.rotary_dim, cr, sr));
                const uint16_t vb = f32_bf16_rne(vr[d]);
                s_new[0][d] = kb;
                s_new[1][d] = vb;
                ((uint16_t *)a.k)[off + d] = kb;
                ((uint16_t *)a.v)[off + d] = vb;
            }
        }
    }

    const float scale = 1.0f / sqrtf((float)HD);
    bf16x8_t qh[NS], ql[NS];
    f32x4 o[NDB];
#pragma unroll
    for (int d = 0; d < NDB; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    const int ntile = (int)((end - start + TW - 1) / TW);
    const int nt = ntile > wave ? (ntile - 1 - wave) / 4 + 1 : 0;  // this wave's tiles
    struct Regs {
        u32x4 k[2][NS];
        u32x4 v[VI];
    };
    // Buffer loads over the tile's valid rows: a row past `end` reads as
    // zeros and moves no memory (its score is masked, its probability 0).
    // Page of tile i (a scalar load), fetched one tile ahead of its use so
    // the lookup does not add a memory round trip before each tile's loads.
    auto page_of = [&](int i) {
        const long t = start + (long)TW * (wave + 4 * min(i, nt - 1));
        return ((const __attribute__((address_space(4))) int32_t *)a.page_table)[t / a.page_size];
    };
    auto load_tile = [&](int i, int page, Regs &R) {
        i = min(i, nt - 1);
        const long t = start + (long)TW * (wave + 4 * i);
        const size_t base = (((size_t)page * a.kv_heads + g) * a.page_size + t % a.page_size) * HD;
        const int valid = (int)min((long)TW, end - t) * ROWB;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void *)((const uint16_t *)a.k + base), (short)0, valid, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void *)((const uint16_t *)a.v + base), (short)0, valid, 0x00020000);
        const int koff = (8 * (n >> 2) + (n & 3)) * ROWB + 16 * kg;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int s = 0; s < NS; ++s)
                R.k[mb][s] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 4 * mb * ROWB + 64 * s, 0, 0));
        const int voff = (lane / CH) * ROWB + 16 * (lane % CH);
#pragma unroll
        for (int i2 = 0; i2 < VI; ++i2)
            R.v[i2] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff, 1024 * i2, 0));
    };
    uint8_t *sv = s_v[wave];
    // First half of a tile: the V tile into this wave's LDS copy and the
    // scores; after it the registers are free for the next tile's loads.
    auto scores = [&](int i, Regs &R, f32x4 (&sc)[2]) {
        if constexpr (ROPE) {
            // The tile holding pos gets the new K/V row (the cache row may
            // not be written yet when the tile was loaded).
            if (has_new && i * 4 + wave == pos_tile) {
                const int rp = (int)(pos - (start + (long)TW * pos_tile));
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const bool mine = 8 * (n >> 2) + 4 * mb + (n & 3) == rp;
#pragma unroll
                    for (int s = 0; s < NS; ++s) {
                        const u32x4 nk = *(const u32x4 *)&s_new[0][32 * s + 8 * kg];
                        R.k[mb][s] = mine ? nk : R.k[mb][s];
                    }
                }
#pragma unroll
                for (int i2 = 0; i2 < VI; ++i2) {
                    const int f = 64 * i2 + lane;
                    const u32x4 nv = *(const u32x4 *)&s_new[1][8 * (f % CH)];
                    R.v[i2] = f / CH == rp ? nv : R.v[i2];
                }
            }
        }
        // V tile into this wave's LDS copy (row f / CH, chunk f % CH).
#pragma unroll
        for (int i2 = 0; i2 < VI; ++i2) {
            const int f = 64 * i2 + lane, r = f / CH, c = f % CH;
            *(u32x4 *)(sv + r * ROWB + 16 * (c ^ vswz<HD>(r))) = R.v[i2];
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const bf16x8_t kA = __builtin_bit_cast(bf16x8_t, R.k[mb][s]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, qh[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kA, ql[s], acc, 0, 0, 0);
            }
            sc[mb] = acc;
        }
    };
    // Second half: online softmax and the value product.
    auto mix = [&](int i, const f32x4 (&sc)[2]) {
        const long t = start + (long)TW * (wave + 4 * i);
        // Online softmax of head n over the tile (positions t + 8kg + 4mb + j).
        float p[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = t + 8 * kg + 4 * mb + j < end;
                const float v = ok ? sc[mb][j] * scale : -INFINITY;
                p[4 * mb + j] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
        float lsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            p[e] = p[e] == -INFINITY ? 0.f : expf(p[e] - m_new);
            lsum += p[e];
        }
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        bf16x8_t ph, pl;
        split_hilo(p, ph, pl);
        // O^T += V^T P^T.
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            s16x4_t h0, h1;
            {
                const int r0 = 8 * kg + (n >> 2), c = 2 * db + ((n & 3) >> 1), b8 = (n & 1) * 8;
                const int r1 = r0 + 4;
                h0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t *)(sv + r0 * ROWB + 16 * (c ^ vswz<HD>(r0)) + b8));
                h1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t *)(sv + r1 * ROWB + 16 * (c ^ vswz<HD>(r1)) + b8));
            }
            const bf16x8_t vA = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7));
            f32x4 acc = o[db] * alpha;
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vA, ph, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vA, pl, acc, 0, 0, 0);
            o[db] = acc;
        }
    };
    // One register set: tile i + 1's loads are issued as soon as tile i's
    // registers have been consumed, and stream in during its softmax and
    // value product (and the other waves' work).
    if (nt > 0) {
        // The group's queries (raw f32 now, converted after the first tile's
        // loads are issued, so the two round trips overlap).
        f32x4 qraw[NS][2];
        // ROPE (rotary width = head_dim): the raw pairs and cos/sin of the
        // lane's 8 dims (all below or all at/above half: multiples of 8).
        f32x4 qpair[ROPE ? NS : 1][4], qcs[ROPE ? NS : 1][4];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            // Every lane loads (lanes past the group re-read head 0 and are
            // zeroed at conversion): no divergent load for the waits to trip on.
            if constexpr (ROPE) {
                const int d0 = 32 * s + 8 * kg;
                const float *src = qkv_row + (size_t)(g * G + (n < G ? n : 0)) * HD;
                const int i0 = d0 < half ? d0 : d0 - half;
#pragma unroll
                for (int k = 0; k < 4; ++k) qpair[s][k] = *(const f32x4 *)(src + 2 * i0 + 4 * k);
                qcs[s][0] = *(const f32x4 *)(cr + i0);
                qcs[s][1] = *(const f32x4 *)(cr + i0 + 4);
                qcs[s][2] = *(const f32x4 *)(sr + i0);
                qcs[s][3] = *(const f32x4 *)(sr + i0 + 4);
            } else {
                const float *qp = a.q + (size_t)row * a.q_stride + (size_t)(g * G + (n < G ? n : 0)) * HD + 32 * s + 8 * kg;
                qraw[s][0] = *(const f32x4 *)qp;
                qraw[s][1] = *(const f32x4 *)(qp + 4);
            }
        }
        const int pg0 = page_of(0);
        int pg_next = page_of(1);
        Regs R;
        load_tile(0, pg0, R);
        __builtin_amdgcn_sched_barrier(0);
        // The queries as the score product's B operand, hi/lo BF16 halves.
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float qv[8];
            const int d0 = 32 * s + 8 * kg;
            if constexpr (ROPE) {
                // rope_elem's arithmetic: a*c - b*s below half, b*c + a*s above.
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float pa = qpair[ROPE ? s : 0][(2 * e) >> 2][(2 * e) & 3];
                    const float pb = qpair[ROPE ? s : 0][(2 * e + 1) >> 2][(2 * e + 1) & 3];
                    const float c = qcs[ROPE ? s : 0][e >> 2][e & 3], sn = qcs[ROPE ? s : 0][2 + (e >> 2)][e & 3];
                    const float r = d0 < half ? pa * c - pb * sn : pb * c + pa * sn;
                    qv[e] = n < G ? r : 0.f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qv[e] = n < G ? qraw[s][0][e] : 0.f;
                    qv[4 + e] = n < G ? qraw[s][1][e] : 0.f;
                }
            }
            split_hilo(qv, qh[s], ql[s]);
        }
        for (int i = 0; i < nt; ++i) {
            f32x4 sc[2];
            scores(i, R, sc);
            const int pg_after = page_of(i + 2);
            load_tile(i + 1, pg_next, R);
            pg_next = pg_after;
            __builtin_amdgcn_sched_barrier(0);
            mix(i, sc);
        }
    }
    // Merge the wave partials in wave order.
    if (n < G) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) s_o[wave][n][16 * db + 4 * kg + j] = o[db][j];
        if (kg == 0) {
            s_m[wave][n] = m_run;
            s_l[wave][n] = l_run;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
        const int j = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][j]);
        float acc = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = s_m[w][j];
            if (mw != -INFINITY) {
                const float sw = expf(mw - M);
                acc = fmaf(sw, s_o[w][j][d], acc);
                L = fmaf(sw, s_l[w][j], L);
            }
        }
        if constexpr (DIRECT) {
            a.out[((size_t)row * a.q_heads + g * G + j) * HD + d] = acc / L;
        } else {
            part[j * part_head + d] = acc;
            if (d == 0) {
                part[j * part_head + HD] = M;
                part[j * part_head + HD + 1] = L;
            }
        }
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
    static_assert(kMaxSplits <= 128, "one wave holds two splits per lane");
    if (tid < 64) {
        const int s1 = tid + 64;
        const float m0 = tid < S ? p[(size_t)tid * (HD + 2) + HD] : -INFINITY;
        const float m1 = s1 < S ? p[(size_t)s1 * (HD + 2) + HD] : -INFINITY;
        const float M = wave_max(fmaxf(m0, m1));
        const float w0 = m0 == -INFINITY ? 0.f : expf(m0 - M);
        const float w1 = m1 == -INFINITY ? 0.f : expf(m1 - M);
        const float l0 = w0 != 0.f ? p[(size_t)tid * (HD + 2) + HD + 1] : 0.f;
        const float l1 = w1 != 0.f ? p[(size_t)s1 * (HD + 2) + HD + 1] : 0.f;
        const float L = wave_sum(w0 * l0) + wave_sum(w1 * l1);
        if (tid < S) s_w[tid] = w0;
        if (s1 < S) s_w[s1] = w1;
        if (tid == 0) s_inv = 1.0f / L;
    }
    __syncthreads();
    const int d = tid % HD, grp = tid / HD;
    // The split values this thread folds are loaded 16 at a time (one memory
    // round trip per batch), then folded in split order.
    constexpr int PER = kMaxSplits / GR, BATCH = PER < 16 ? PER : 16;
    float o = 0.f;
    for (int i0 = 0; i0 < PER && grp + GR * i0 < S; i0 += BATCH) {
        float v[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int s = grp + GR * (i0 + i);
            v[i] = s < S ? p[(size_t)s * (HD + 2) + d] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int s = grp + GR * (i0 + i);
            const float w = s < S ? s_w[s] : 0.f;
            if (w != 0.f) o = fmaf(w, v[i], o);
        }
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

// ---------------------------------------------------------------------------
// Chunked prefill on the matrix cores (BF16 KV): flash attention with the
// score and value products as v_mfma_f32_32x32x16_bf16.
//
// A block is 4 waves and one KV head; each wave owns 32 "M rows" = RW query
// rows x G heads of the group (RW = 32 / G). Per 64-position tile:
//   S^T = K Q^T  (A = K rows from LDS, B = Q^T kept in registers as hi/lo
//                BF16 halves of the f32 query, so scores carry ~2^-17
//                relative error); every lane ends up holding one M row's
//                scores (column = lane % 32), so the online softmax (running
//                max / sum, rescale) is lane-local plus one exchange with
//                lane ^ 32.
//   O^T += V^T P^T (A = V^T from LDS, B = P^T straight from the S^T
//                registers, again as hi/lo BF16 halves).
// K rows are staged in LDS with bits 2 and 3 of the position swapped, which
// makes the S^T output registers exactly the B operand layout of the second
// product (8 consecutive positions per lane), so P never moves between lanes.
// V is staged transposed ([dim][position]).
//
// Splits are absolute position ranges of `span` keys (fixed per model), so
// every row's result depends only on its own position (the same bits however
// the prompt is chunked); the splits of a row are merged in order by
// attn_merge2_kernel.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// LDS row of a position within a 64-position tile (an involution).
__device__ __forceinline__ int krow_of(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }

// hi = bf16(v) and lo = bf16(v - hi) (hardware round-to-nearest-even
// conversions), so hi + lo carries v to ~2^-17 relative error.
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        hi[q] = (__bf16)v[q];
        lo[q] = (__bf16)(v[q] - (float)hi[q]);
    }
}

// Column of position p (0..63) in row d of the transposed V tile: groups of 8
// positions are XOR-swizzled by the row's dim group, so the transposing
// stores of one wave spread over the LDS banks while every 8-position group
// stays one aligned 16-byte read.
__device__ __forceinline__ int vcol(int d, int p) { return (((p >> 3) ^ ((d >> 3) & 7)) << 3) | (p & 7); }

template <int HD, int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill_kernel(AttnArgs a, int rows, int S, int span) {
    constexpr int RW = 32 / G, MV = RW * G;
    constexpr int LDV = 64 + 8;
    constexpr int KSTEPS = HD / 16, UT = HD / 32, KC = HD / 32;
    constexpr int CPR = HD / 8;  // 16-byte chunks per K row
    // K rows unpadded, chunk c of LDS row r stored at chunk c ^ (r % CPR).
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][64 * HD];
    __shared__ __attribute__((aligned(16))) uint16_t vt[2][HD * LDV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, half = lane >> 5;
    const int rb = blockIdx.x, g = blockIdx.y, split = blockIdx.z;
    const int row = rb * 4 * RW + wave * RW + n / G;
    const int head = g * G + n % G;
    const bool rvalid = n < MV && row < rows;
    // Positions fit in 32 bits (the KV capacity is checked on the host).
    const int off = (int)a.offset;
    const int my_pos = off + row;
    const int first_pos = off + rb * 4 * RW;
    const int ctx = off + min(rows, (rb + 1) * 4 * RW);
    const int start = split * span;
    const int end = min(start + span, ctx);
    float *part = a.part + (((size_t)row * a.q_heads + head) * S + split) * (HD + 2);
    if (start >= ctx) {  // block-uniform: no row of this block reaches the split
        if (rvalid && half == 0) part[HD] = -INFINITY;
        return;
    }

    // Q^T operands (B of S^T = K Q^T): lane holds Q[m = lane % 32][16 s + 8 half .. +8],
    // pre-scaled by log2(e) / sqrt(HD) so scores come out in the exp2 domain.
    bf16x8 qh[KSTEPS], ql[KSTEPS];
    {
        const float sl2 = (1.0f / sqrtf((float)HD)) * 1.44269504088896340736f;
        const float *qp = a.q + (size_t)(rvalid ? row : 0) * a.q_stride + (size_t)head * HD + 8 * half;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (rvalid) {
                const f32x4 t0 = *(const f32x4 *)(qp + 16 * s), t1 = *(const f32x4 *)(qp + 16 * s + 4);
                v[0] = t0[0] * sl2; v[1] = t0[1] * sl2; v[2] = t0[2] * sl2; v[3] = t0[3] * sl2;
                v[4] = t1[0] * sl2; v[5] = t1[1] * sl2; v[6] = t1[2] * sl2; v[7] = t1[3] * sl2;
            }
            split8(v, qh[s], ql[s]);
        }
    }

    const uint16_t *kbase = (const uint16_t *)a.k, *vbase = (const uint16_t *)a.v;
    u32x4 vr[KC];
    // K: direct global->LDS copies. One wave instruction fills 1 KB = 64 / CPR
    // LDS rows; lane i lands at byte 16 i, so it fetches the global chunk
    // that the swizzle places there. Rows past the split end may hold stale
    // bytes: their scores are masked before use.
    auto fetch_k = [&](int t0, int b) {
        const int page = a.page_table[t0 / a.page_size];
        const size_t tile = (((size_t)page * a.kv_heads + g) * a.page_size + (t0 % a.page_size)) * HD;
        constexpr int RPI = 64 / CPR;  // LDS rows per wave instruction
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int r0 = (wave + 4 * c) * RPI;  // first LDS row of this instruction
            const int r = r0 + lane / CPR, cs = lane % CPR;
            const int p = krow_of(r), chunk = cs ^ (r % CPR);
            __builtin_amdgcn_global_load_lds(kbase + tile + (size_t)p * HD + chunk * 8,
                                             (__attribute__((address_space(3))) void *)(&ks[b][r0 * HD]), 16, 0, 0);
        }
    };
    auto fetch_v = [&](int t0) {
        const int page = a.page_table[t0 / a.page_size];
        const size_t tile = (((size_t)page * a.kv_heads + g) * a.page_size + (t0 % a.page_size)) * HD;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int idx = tid + kThreads * c, p = idx / CPR, d0 = (idx % CPR) * 8;
            // positions past the split end may be unwritten: zeros (p = 0 there)
            vr[c] = t0 + p < end ? *(const u32x4 *)(vbase + tile + p * HD + d0) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_v = [&](int b) {
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int idx = tid + kThreads * c, p = idx / CPR, d0 = (idx % CPR) * 8;
            const int col = vcol(d0, p);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                vt[b][(d0 + e) * LDV + col] = (uint16_t)((e & 1) ? (vr[c][e >> 1] >> 16) : (vr[c][e >> 1] & 0xFFFFu));
        }
    };

    f32x16 oacc[UT];
#pragma unroll
    for (int u = 0; u < UT; ++u) oacc[u] = f32x16{};
    float m2 = -INFINITY, l = 0.f;
    fetch_k(start, 0);
    fetch_v(start);
    store_v(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int b = 0;
    for (int t0 = start; t0 < end; t0 += 64) {
        const bool more = t0 + 64 < end;
        if (more) {
            fetch_k(t0 + 64, b ^ 1);
            fetch_v(t0 + 64);
        }
        // Two halves of 32 positions, each: S^T, online softmax, O^T update.
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            f32x16 sacc = f32x16{};
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const int r = 32 * tt + n;
                const bf16x8 ka =
                    __builtin_bit_cast(bf16x8, *(const u32x4 *)(&ks[b][r * HD + (((2 * s + half) ^ (r % CPR)) << 3)]));
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qh[s], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, ql[s], sacc, 0, 0, 0);
            }
            // Causal / split-end mask, only where the half reaches past a
            // row's position or past the split (block-uniform test).
            const int h0 = t0 + 32 * tt;
            if (h0 + 31 > first_pos || h0 + 32 > end) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int p = h0 + krow_of(8 * (r >> 2) + 4 * half + (r & 3));
                    if (p > my_pos || p >= end) sacc[r] = -INFINITY;
                }
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[r]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            // Delayed rescaling: exponentials are taken against a reference
            // max m2 that is raised only when a score exceeds it by more than
            // 8 (log2 units), so p <= 256 and the O / l rescale is rare. Each
            // row's steps depend only on its own scores.
            const bool raise = tmax > m2 + 8.0f;
            if (__any(raise)) {
                const float mnew = raise ? tmax : m2;
                const float alpha = __builtin_amdgcn_exp2f(m2 - mnew);  // 1 where not raised, 0 from -inf
                l *= alpha;
#pragma unroll
                for (int u = 0; u < UT; ++u)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[u][r] *= alpha;
                m2 = mnew;
            }
            // A row with every score so far masked keeps m2 = -inf; its terms are 0.
            const float mref = m2 == -INFINITY ? 0.f : m2;
            float tsum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = __builtin_amdgcn_exp2f(sacc[r] - mref);
                sacc[r] = pv;
                tsum += pv;
            }
            tsum += __shfl_xor(tsum, 32, 64);
            l += tsum;
            // O^T += V^T P^T over 2 steps of 16 positions.
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                float pv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) pv[j] = sacc[8 * s2 + j];
                bf16x8 bh, bl;
                split8(pv, bh, bl);
#pragma unroll
                for (int u = 0; u < UT; ++u) {
                    const int d = 32 * u + n;
                    const bf16x8 va = __builtin_bit_cast(
                        bf16x8, *(const u32x4 *)(&vt[b][d * LDV + vcol(d, 32 * tt + 16 * s2 + 8 * half)]));
                    oacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, bh, oacc[u], 0, 0, 0);
                    oacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, bl, oacc[u], 0, 0, 0);
                }
            }
        }
        if (more) store_v(b ^ 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        b ^= 1;
    }
    if (!rvalid) return;
    // O^T registers: lane's M row, dims 32 u + 8 (r / 4) + 4 half + r % 4.
    if (S == 1) {
        const float inv = 1.0f / l;
        const size_t ob = (size_t)row * (size_t)a.q_heads * HD + (size_t)head * HD;
        float *o = a.out + ob;
#pragma unroll
        for (int u = 0; u < UT; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = f32x4{oacc[u][4 * q] * inv, oacc[u][4 * q + 1] * inv, oacc[u][4 * q + 2] * inv,
                                      oacc[u][4 * q + 3] * inv};
                *(f32x4 *)(o + 32 * u + 8 * q + 4 * half) = v;
                if (a.out_hi) store_halves4(a.out_hi, a.out_lo, ob + 32 * u + 8 * q + 4 * half, v);
            }
    } else {
#pragma unroll
        for (int u = 0; u < UT; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(f32x4 *)(part + 32 * u + 8 * q + 4 * half) =
                    f32x4{oacc[u][4 * q], oacc[u][4 * q + 1], oacc[u][4 * q + 2], oacc[u][4 * q + 3]};
        if (half == 0) {
            part[HD] = m2;
            part[HD + 1] = l;
        }
    }
}

// Merges the splits of one (row, q head) of attn_prefill_kernel in split
// order, one wave per (row, head): maxima in the log2 domain, weights
// 2^(m_s - M), output (sum_s w_s o_s) * (1 / sum_s w_s l_s). A row whose only
// non-empty split gives w = 1 gets o * (1 / l), the bits the one-split
// kernel writes.
template <int HD>
__global__ __launch_bounds__(kThreads) void attn_merge2_kernel(const float *part, int S, int q_heads, int items,
                                                              float *out, uint16_t *out_hi, uint16_t *out_lo) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (item >= items) return;
    const float *p = part + (size_t)item * (size_t)S * (HD + 2);
    const float m = lane < S ? p[(size_t)lane * (HD + 2) + HD] : -INFINITY;
    const float M = wave_max(m);
    const float w = m == -INFINITY ? 0.f : exp2f(m - M);
    const float L = wave_sum(w != 0.f ? w * p[(size_t)lane * (HD + 2) + HD + 1] : 0.f);
    const float inv = 1.0f / L;
    constexpr int DPL = HD / 64;  // dims per lane
    float o[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) o[k] = 0.f;
    for (int s = 0; s < S; ++s) {
        const float ws = __shfl(w, s, 64);
        if (ws != 0.f) {
#pragma unroll
            for (int k = 0; k < DPL; ++k) o[k] = fmaf(ws, p[(size_t)s * (HD + 2) + lane + 64 * k], o[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
        const size_t i = (size_t)item * HD + lane + 64 * k;
        const float v = o[k] * inv;
        out[i] = v;
        if (out_hi) {
            const __bf16 hb = (__bf16)v;
            out_hi[i] = __builtin_bit_cast(uint16_t, hb);
            out_lo[i] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)hb));
        }
    }
}

template <int HD, int G>
int launch_prefill_hg(const AttnJob &j, const AttnArgs &a, int S, hipStream_t s) {
    constexpr int RW = 32 / G;
    const int rb = (int)((j.rows + 4 * RW - 1) / (4 * RW));
    hipLaunchKernelGGL((attn_prefill_kernel<HD, G>), dim3(rb, j.g.kv_heads, S), dim3(kThreads), 0, s, a, (int)j.rows,
                       S, j.span);
    CHIP_CHECK(hipGetLastError());
    if (S > 1) {
        const int items = (int)j.rows * j.q_heads;
        hipLaunchKernelGGL((attn_merge2_kernel<HD>), dim3((items + 3) / 4), dim3(kThreads), 0, s, a.part, S,
                           j.q_heads, items, a.out, a.out_hi, a.out_lo);
        CHIP_CHECK(hipGetLastError());
    }
    return 0;
}

template <int HD>
int launch_prefill_h(const AttnJob &j, const AttnArgs &a, int G, int S, hipStream_t s) {
    switch (G) {
        case 1: return launch_prefill_hg<HD, 1>(j, a, S, s);
        case 2: return launch_prefill_hg<HD, 2>(j, a, S, s);
        case 3: return launch_prefill_hg<HD, 3>(j, a, S, s);
        case 4: return launch_prefill_hg<HD, 4>(j, a, S, s);
        case 5: return launch_prefill_hg<HD, 5>(j, a, S, s);
        case 6: return launch_prefill_hg<HD, 6>(j, a, S, s);
        case 7: return launch_prefill_hg<HD, 7>(j, a, S, s);
        case 8: return launch_prefill_hg<HD, 8>(j, a, S, s);
    }
    return fail("HIP backend: attention supports 1..8 query heads per KV head.");
}

// Decode attention: BF16 K/V on the matrix cores, f32 K/V on the vector
// ALUs.
template <int HD, int G, class KT>
int launch_hgk(const AttnJob &j, const AttnArgs &a, hipStream_t s) {
    const dim3 grid(j.splits, j.g.kv_heads, j.rows);
    constexpr bool mfma = std::is_same<KT, uint16_t>::value;
    const bool rope = a.qkv != nullptr;
    if (rope && !mfma) return fail("HIP backend: fused RoPE needs the matrix-core attention kernel.");
    if (j.splits == 1) {
        if constexpr (mfma) {
            if (rope) hipLaunchKernelGGL((attn_dec_mfma_kernel<HD, G, true, true>), grid, dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((attn_dec_mfma_kernel<HD, G, true, false>), grid, dim3(kThreads), 0, s, a);
        } else {
            hipLaunchKernelGGL((attn_kernel<HD, G, KT, true>), grid, dim3(kThreads), 0, s, a);
        }
        CHIP_CHECK(hipGetLastError());
        return 0;
    }
    if constexpr (mfma) {
        if (rope) hipLaunchKernelGGL((attn_dec_mfma_kernel<HD, G, false, true>), grid, dim3(kThreads), 0, s, a);
        else hipLaunchKernelGGL((attn_dec_mfma_kernel<HD, G, false, false>), grid, dim3(kThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL((attn_kernel<HD, G, KT, false>), grid, dim3(kThreads), 0, s, a);
    }
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

// Split-K of a decode-style launch: across the KV heads and rows about one
// block per CU for the matrix-core kernel (BF16 K/V; measured 13 % faster
// than two at 16K keys, where the K/V stream, not the block count, sets the
// time) and two for the VALU kernel (f32 K/V), at most one split per
// 64-position tile and kMaxSplits.
int attention_decode_splits(size_t ctx, int kv_heads, size_t rows, bool kv_f32) {
    const size_t per_cu = kv_f32 ? 2 : 1;
    const size_t target = per_cu * (size_t)std::max(device_cus(), 1);
    const size_t per = (size_t)std::max(kv_heads, 1) * std::max<size_t>(rows, 1);
    size_t s = (target + per - 1) / per;
    s = std::min({s, (ctx + TP - 1) / TP, (size_t)kMaxSplits});
    return (int)std::max<size_t>(s, 1);
}

int attention_prefill_splits(size_t ctx, int span) {
    return (int)std::max<size_t>(1, (ctx + (size_t)span - 1) / (size_t)span);
}

// Longer spans mean fewer splits to merge per row and fewer, larger blocks:
// measured on 1,024-row chunks at up to 32K keys (Qwen2-7B turn 1 / turn 2
// prefill) 19,130 / 14,155 tok/s with 1,024, 20,418 / 15,737 with 4,096;
// on 512-row chunks at up to 8K keys (Llama-3-8B) 20,766 tok/s with 1,024,
// 19,178 with 4,096. Capacity / 8 picks 4,096 for the 33K cache and 1,024
// for the 8K one.
int attention_prefill_span(size_t kv_capacity) {
    int span = kDefaultPrefillSpan;
    while ((size_t)span * 2 <= kv_capacity / 8 && span < (1 << 20)) span *= 2;
    return span;
}

bool attention_decode_fuses_rope(const KvGeom &g, int q_heads, int rotary_dim) {
    return !g.kv_f32 && (g.head_dim == 64 || g.head_dim == 128) && g.kv_heads > 0 &&
           q_heads % g.kv_heads == 0 && q_heads / g.kv_heads <= 8 && rotary_dim == g.head_dim;
}

bool attention_prefill_on_mfma(const KvGeom &g, int q_heads) {
    return !g.kv_f32 && (g.head_dim == 64 || g.head_dim == 128) && g.kv_heads > 0 && q_heads % g.kv_heads == 0 &&
           q_heads / g.kv_heads <= 8;
}

int launch_attention(const AttnJob &j, hipStream_t s) {
    if (j.rows == 0) return 0;
    if ((!j.q && !j.qkv) || !j.out || !j.k || !j.v || !j.g.page_table || (!j.prefill && j.splits > 1 && !j.part))
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
    if (j.qkv) {
        if (j.prefill || j.rows != 1 || !attention_decode_fuses_rope(j.g, j.q_heads, j.rotary_dim) || !j.rope_cos ||
            !j.rope_sin)
            return fail("HIP backend: fused RoPE attention takes one BF16 decode row with full-width rotary.");
        a.qkv = j.qkv;
        a.rope_cos = j.rope_cos;
        a.rope_sin = j.rope_sin;
        a.rotary_dim = j.rotary_dim;
    }
    const int G = j.q_heads / j.g.kv_heads;
    if (j.prefill && attention_prefill_on_mfma(j.g, j.q_heads)) {
        if (j.pos_dev) return fail("HIP backend: prefill attention takes a host position.");
        if (j.offset + j.rows > (size_t)INT32_MAX) return fail("HIP backend: prefill position out of range.");
        if (j.span < 64 || j.span % 64) return fail("HIP backend: prefill span must be a positive multiple of 64.");
        const int S = attention_prefill_splits(j.offset + j.rows, j.span);
        if (S > kMaxSplits) return fail("HIP backend: prefill context exceeds the attention split limit.");
        if (S > 1 && (!j.part || j.part_floats < attention_part_floats(j.rows, j.q_heads, S, j.g.head_dim)))
            return fail("HIP backend: prefill attention partial buffer too small.");
        if (!j.out_hi != !j.out_lo || ((uintptr_t)j.out_hi % 8) || ((uintptr_t)j.out_lo % 8))
            return fail("HIP backend: prefill attention halves need both 8-byte aligned buffers.");
        a.out_hi = j.out_hi;
        a.out_lo = j.out_lo;
        if (j.g.head_dim == 64) return launch_prefill_h<64>(j, a, G, S, s);
        return launch_prefill_h<128>(j, a, G, S, s);
    }
    if (j.g.head_dim == 64) return launch_h<64>(j, a, G, s);
    if (j.g.head_dim == 128) return launch_h<128>(j, a, G, s);
    return fail("HIP backend: attention supports head_dim 64 and 128.");
}

}  // namespace chip
