// Persistent dataflow decode kernel: one cooperative launch (one 512-thread
// block per CU) runs whole decode steps -- embedding, every layer, LM head,
// greedy argmax -- with no device-wide barrier.
//
// Per layer five phases, per step one more:
//   A  QKV rows (fused RMSNorm, bias, RoPE); K/V rows appended to the pages
//   B  GQA attention: one item = (KV head, run of positions), two-pass softmax
//   C  attention partials merged in split order, o_proj + residual
//   D  gate/up (fused RMSNorm) + SwiGLU
//   E  down + residual
//   H  LM head (fused final RMSNorm) + per-block argmax partials; blocks that
//      need the next token reduce all partials themselves (ties to the last
//      index, engine.rs:2247-2253)
//
// Phases are chained through the data. Every value one block hands to
// another is a 64-bit word {f32 bits, tag}, where the tag names the phase
// instance that produced it (launch base + step * (5L + 1) + 5 * layer +
// phase). A consumer copies the words it needs into LDS with direct
// global->LDS loads (16 bytes per lane, device-coherent sc1, many in flight,
// no registers), checks the tags there, and re-loads only the 128-word
// chunks that are still stale; aligned 8-byte stores are single-copy atomic,
// so value and tag arrive together. A phase therefore starts as soon as its
// own inputs exist. Producers write with device-scope relaxed atomic stores
// (sc1), coherent across the XCDs' separate L2 caches, and so are the K/V
// pages, which attention reads the same way into LDS. Weights are read-only
// and use plain non-temporal loads.
//
// Each wave owns fixed rows of every projection and issues the loads of a
// phase's weight rows into registers before it polls that phase's inputs,
// so HBM streaming overlaps the wait for the producers.
//
// Buffer reuse needs no barrier: a block polls a phase's inputs only in a
// phase where it also produces outputs, and every buffer is rewritten only by
// a phase that transitively depends on all of those outputs. Only blocks
// that own LM-head rows (and so wait for the final hidden state) write
// argmax partials; those alternate between two buffers by step parity.
//
// Every poll is bounded: on timeout a block raises the abort word, which all
// polls watch, and every wave returns; the host then resets the tagged words.
//
// Math per phase is that of the multi-kernel path (gemv.hip, attention.hip,
// misc.hip), i.e. the reference path of ops.rs / qwen2.rs; only f32
// summation orders differ.
#include <cstdlib>

#include "decode_fused.hpp"
#include "wunit.hpp"

namespace chip {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int TP = 64;            // positions per KV page
constexpr int kChunk = 128;       // tagged words per wave-wide 16-byte-per-lane load
constexpr int kLdsBudget = 128 * 1024;  // dynamic LDS the layout may use
constexpr long kSpinLimit = 1L << 20;

// threadIdx.x through an opaque copy: address arithmetic stays next to its
// use inside the step loop instead of being hoisted out of it and held in
// registers for the whole kernel.
__device__ __forceinline__ int tid_here() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// Global wave index, recomputed where used (same reason).
__device__ __forceinline__ int gw_here() { return (int)blockIdx.x * kWaves + (tid_here() >> 6); }

__device__ __forceinline__ void stt(uint64_t *p, uint32_t bits, unsigned tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf(uint64_t *p, float v, unsigned tag) { stt(p, __float_as_uint(v), tag); }
__device__ __forceinline__ unsigned tag_of(uint64_t w) { return (unsigned)(w >> 32); }
__device__ __forceinline__ float val_of(uint64_t w) { return __uint_as_float((uint32_t)w); }

__device__ __forceinline__ void st_kv(uint16_t *p, float v) {
    __hip_atomic_store(p, f32_bf16_rne(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_kv(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The value a K/V element has once stored in the cache.
template <class KT>
__device__ __forceinline__ float kv_round(float v) {
    if constexpr (sizeof(KT) == 2) return bf16_f32(f32_bf16_rne(v));
    else return v;
}

__device__ __forceinline__ bool aborted(const int *f) {
    return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void raise_abort(int *f) {
    __hip_atomic_store(f, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One layer's pointer table by value, read through the constant address
// space: scalar loads into scalar registers, not re-read after every store
// (a reference into global memory would be, as the stores might alias it).
__device__ __forceinline__ FusedLayer load_layer(const FusedLayer *table, int l) {
    typedef const __attribute__((address_space(4))) FusedLayer CLayer;
    CLayer *p = (CLayer *)table + l;
    FusedLayer o;
    o.qkv = p->qkv;
    o.o = p->o;
    o.gate = p->gate;
    o.up = p->up;
    o.down = p->down;
    o.qkv_sc = p->qkv_sc;
    o.o_sc = p->o_sc;
    o.gate_sc = p->gate_sc;
    o.up_sc = p->up_sc;
    o.down_sc = p->down_sc;
    o.qkv_bias = p->qkv_bias;
    o.o_bias = p->o_bias;
    o.ln1 = p->ln1;
    o.ln2 = p->ln2;
    o.kc = p->kc;
    o.vc = p->vc;
    return o;
}

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (lds must be the same in every lane of the wave), device-coherent (sc1).
__device__ __forceinline__ void dma16(const void *g, void *lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds, 16, 0, 16);
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Copies tagged words src[0, n) into LDS dst[0, n) and waits until each
// carries `tag`. Wave w loads chunks w, w + 4, ... (128 words each); after
// each round only chunks with a stale word are loaded again. Block-wide:
// starts with a barrier (dst may still be read by the previous phase) and
// ends with one; false in every thread on timeout or abort.
__device__ __forceinline__ bool gather_lds(uint64_t *dst, const uint64_t *src, int n, unsigned tag, int *abort_flag) {
    const int tid = tid_here(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int chunks = (n + kChunk - 1) / kChunk;
    __syncthreads();
    uint64_t pend = 0;  // bit i: chunk wave + 4 i is stale
    for (int c = wave, i = 0; c < chunks; c += kWaves, ++i) pend |= 1ull << i;
    long spins = 0;
    bool ok = true;
    while (pend) {
        for (int c = wave, i = 0; c < chunks; c += kWaves, ++i)
            if ((pend >> i) & 1) {
                const int w = c * kChunk + lane * 2;
                if (w < n) dma16(src + w, dst + c * kChunk);
            }
        wait_dma();
        uint64_t still = 0;
        for (int c = wave, i = 0; c < chunks; c += kWaves, ++i)
            if ((pend >> i) & 1) {
                const int w = c * kChunk + lane * 2;
                bool stale = w < n && tag_of(dst[w]) != tag;
                stale |= w + 1 < n && tag_of(dst[w + 1]) != tag;
                if (__any(stale)) still |= 1ull << i;
            }
        pend = still;
        if (pend) {
            if (++spins > kSpinLimit || ((spins & 15) == 0 && aborted(abort_flag))) {
                raise_abort(abort_flag);
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    return __syncthreads_and(ok);
}

// xs[i] = value of tb[i] (i < n); with a gain, RMSNorm'd in place as the
// GEMV prologue does: x * (inv * g), inv = 1 / sqrt(mean(x^2) + eps)
// (ops.rs:646-652). Block-wide; ends with a barrier.
__device__ void stage_lds(float *xs, const uint64_t *tb, int n, const uint16_t *gain, float eps, float *red) {
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
    for (int i = tid; i < n; i += kThreads) {
        const float v = val_of(tb[i]);
        xs[i] = v;
        ss = fmaf(v, v, ss);
    }
    if (gain) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total += red[w];
        const float inv = 1.0f / sqrtf(total / (float)n + eps);
        for (int i = tid; i < n; i += kThreads) xs[i] = xs[i] * (inv * bf16_f32(gain[i]));
    }
    __syncthreads();
}

// The embedding row, RMSNorm'd (layer 0's QKV input).
__device__ void stage_embed(float *xs, const uint16_t *row, int n, const uint16_t *gain, float eps, float *red) {
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
    for (int i = tid; i < n; i += kThreads) {
        const float v = bf16_f32(row[i]);
        xs[i] = v;
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) total += red[w];
    const float inv = 1.0f / sqrtf(total / (float)n + eps);
    for (int i = tid; i < n; i += kThreads) xs[i] = xs[i] * (inv * bf16_f32(gain[i]));
    __syncthreads();
}

// One weight row as 16-byte units, unit u in lane u % 64, slot u / 64.
template <int N>
__device__ __forceinline__ void load_row(u32x4 (&w)[N], const uint8_t *row, int n_units) {
    const int lane = tid_here() & 63;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = lane + 64 * k;
        if (u < n_units) w[k] = __builtin_nontemporal_load((const u32x4 *)(row + (size_t)u * 16));
    }
}

// Wave-wide dot products of R loaded rows (the first nr valid, nr uniform
// across the wave) with xs; a unit's x values are read once for all rows.
// Per row the summation order is fixed (unit, then element). Results land
// in every lane.
template <int FMT, int R, int N>
__device__ __forceinline__ void dot_rows(const u32x4 (&w)[R][N], const float *xs, int n_units, int nr,
                                         float (&out)[R]) {
    using U = Unit<FMT, 16>;
    const int lane = tid_here() & 63;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = lane + 64 * k;
        if (u < n_units) {
            float xv[U::E];
#pragma unroll
            for (int e = 0; e < U::E; ++e) xv[e] = xs[u * U::E + e];
#pragma unroll
            for (int i = 0; i < R; ++i)
                if (i < nr) {
                    const uint32_t raw[4] = {w[i][k][0], w[i][k][1], w[i][k][2], w[i][k][3]};
                    U::decode(raw, [&](int e, float v) { acc[i] = fmaf(v, xv[e], acc[i]); });
                }
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) out[i] = i < nr ? wave_sum(acc[i]) : 0.f;
}

__device__ __forceinline__ int total_key(float f) {
    const int i = __float_as_int(f);
    return i ^ (int)(((unsigned)(i >> 31)) >> 1);
}
__device__ __forceinline__ void better(int &key, uint32_t &idx, int k2, uint32_t i2) {
    if (k2 > key || (k2 == key && i2 > idx)) {
        key = k2;
        idx = i2;
    }
}

constexpr int kStage = 64;  // outputs one block publishes per phase, at most

struct Shm {
    float red[kWaves];
    int ikey[kWaves];
    uint32_t iidx[kWaves];
    // A phase's outputs of the block's waves, stored by one wave afterwards
    // so that consecutive words leave in one coalesced run.
    float outv[kStage];
    int outi[kStage];   // destination word (QKV: index into the q/K/V words)
    int outc[kStage];   // QKV: cache element (bit 30: V cache), or -1
};

// Stores vals[0, n) as the tagged words dst[0, n): one run by the first
// threads. Block-wide; starts with a barrier (the values are staged by other
// waves).
__device__ __forceinline__ void publish(uint64_t *dst, const float *vals, int n, unsigned tag) {
    __syncthreads();
    const int tid = tid_here();
    if (tid < n) stf(dst + tid, vals[tid], tag);
}

// Reduces (key, idx) over the block; the result lands in every thread.
__device__ void block_best(int &key, uint32_t &idx, Shm &sm) {
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int k2 = __shfl_xor(key, off, 64);
        const uint32_t i2 = __shfl_xor(idx, off, 64);
        better(key, idx, k2, i2);
    }
    if (lane == 0) {
        sm.ikey[wave] = key;
        sm.iidx[wave] = idx;
    }
    __syncthreads();
    key = sm.ikey[0];
    idx = sm.iidx[0];
    for (int w = 1; w < kWaves; ++w) better(key, idx, sm.ikey[w], sm.iidx[w]);
    __syncthreads();
}

// Attention work-item geometry: T threads per position (8 elements each),
// P positions per pass, CH positions per item (one 64-position page: many
// small items keep each block's share of the attention short).
template <int HD, class KT>
struct AttnGeo {
    static constexpr int T = HD / 8;
    static constexpr int P = kThreads / T;
    static constexpr int ROW = HD * (int)sizeof(KT);  // bytes of one K or V row
    static constexpr int CH = TP;
};

template <int HD, int G, int CH>
struct AttnShm {
    static constexpr int GP = (G + 3) / 4 * 4;
    float p[CH][GP];  // scores, then weights, of position x head
    float red[kWaves][G][HD];
    float m[G], l[G];
};

__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Dynamic LDS layout (byte offsets): tagged-word staging, the f32 vector,
// merge weights. The staging area also holds one attention item's q/K/V:
// the group's q and new K/V words first, then its K rows and V rows.
struct LdsLayout {
    int qkw;    // words reserved for a group's q + new K/V
    int tbw;    // staging words
    int xs, total;
};
__host__ __device__ inline LdsLayout lds_layout(int H, int I, int nq, int hd, int G, int kv_bytes, int blocks,
                                                int max_splits) {
    LdsLayout o{};
    o.qkw = round_up((G + 2) * hd, kChunk);
    int tbw = o.qkw + 2 * TP * hd * kv_bytes / 8;
    tbw = tbw > H ? tbw : H;
    tbw = tbw > I ? tbw : I;
    tbw = tbw > 2 * blocks ? tbw : 2 * blocks;
    const int parts = max_splits * G * (hd + 2);
    tbw = tbw > parts ? tbw : parts;
    o.tbw = round_up(tbw + 2, kChunk);
    int xf = H > I ? H : I;
    xf = xf > nq * hd ? xf : nq * hd;
    o.xs = o.tbw * 8;
    o.total = o.xs + xf * 4;
    return o;
}

// Loads the cached K and V rows of positions [start, lim) of KV head g into
// LDS (row p - start of each), 64-position pages at a time.
template <int HD, class KT>
__device__ void load_kv_lds(uint8_t *k_lds, uint8_t *v_lds, const FusedArgs &a, const FusedLayer &ly, int g,
                            long start, long lim) {
    using Geo = AttnGeo<HD, KT>;
    const int tid = tid_here(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int NT = Geo::CH / TP;
    int pages[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) pages[t] = start + t * TP < lim ? a.page_table[(start + t * TP) / TP] : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const long t0 = start + t * TP;
        if (t0 >= lim) break;
        const int page = pages[t];
        const int bytes = (int)(min((long)TP, lim - t0)) * Geo::ROW;
        const size_t off = (((size_t)page * a.kv_heads + g) * TP) * Geo::ROW;
        const uint8_t *ks = (const uint8_t *)ly.kc + off, *vs = (const uint8_t *)ly.vc + off;
        uint8_t *kd = k_lds + (t0 - start) * Geo::ROW, *vd = v_lds + (t0 - start) * Geo::ROW;
        for (int c = wave * 1024; c < bytes; c += kWaves * 1024) {
            const int byte = c + lane * 16;
            if (byte < bytes) {
                dma16(ks + byte, kd + c);
                dma16(vs + byte, vd + c);
            }
        }
    }
}

template <class KT>
__device__ __forceinline__ void ld8(const KT *p, float (&f)[8]) {
    if constexpr (sizeof(KT) == 2) {
        const u32x4 v = *(const u32x4 *)p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = bf16_lo(v[i]);
            f[2 * i + 1] = bf16_hi(v[i]);
        }
    } else {
        const f32x4 a = *(const f32x4 *)p, b = *(const f32x4 *)(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = a[i];
            f[4 + i] = b[i];
        }
    }
}

// Attention item (KV head g, positions [split * CH, ...)) for all G heads of
// the group; writes (unnormalised output, max, sum) partials per q head.
// With `late`, the cached rows are loaded only after the q gather (whose
// tags prove every earlier position of this layer is written); otherwise
// they were loaded into LDS beforehand.
template <int HD, int G, class KT>
__device__ bool attn_item(const FusedArgs &a, const FusedLayer &ly, uint64_t *tb, int g, int split, int S, long pos,
                          unsigned tA, unsigned tB, bool late, int qkw,
                          AttnShm<HD, G, AttnGeo<HD, KT>::CH> &sh, uint64_t *tr) {
    using Geo = AttnGeo<HD, KT>;
    constexpr int T = Geo::T, P = Geo::P, CH = Geo::CH;
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    const int d8 = tid % T, pg = tid / T;
    auto mark = [&](int ev) {
        if (tr && tid == 0) tr[ev] = wall_clock64();
    };
    const long ctx = pos + 1;
    const long start = (long)split * CH;
    const long end = min(start + CH, ctx);
    const int nv = (int)(end - start);
    uint8_t *k_lds = (uint8_t *)(tb + qkw), *v_lds = k_lds + CH * Geo::ROW;
    if (!gather_lds(tb, a.qkvn + (size_t)g * (G + 2) * HD, (G + 2) * HD, tA, a.abort_flag)) return false;
    if (late) {
        load_kv_lds<HD, KT>(k_lds, v_lds, a, ly, g, start, min(end, pos));
        wait_dma();
        __syncthreads();
    }
    if (end == ctx) {
        // The new position's K and V rows, as stored in the cache.
        for (int i = tid; i < 2 * HD; i += kThreads) {
            const float v = val_of(tb[G * HD + i]);
            KT *row = (KT *)((i < HD ? k_lds : v_lds) + (size_t)(nv - 1) * Geo::ROW);
            if constexpr (sizeof(KT) == 2) row[i % HD] = f32_bf16_rne(v);
            else row[i % HD] = v;
        }
        __syncthreads();
    }
    mark(0);
    // q as f32 in LDS (reusing the staging words it came in).
    float *qs = (float *)tb;
    __syncthreads();
    {
        float qv[(G * HD + kThreads - 1) / kThreads];
#pragma unroll
        for (int k = 0; k * kThreads < G * HD; ++k)
            if (tid + k * kThreads < G * HD) qv[k] = val_of(tb[tid + k * kThreads]);
        __syncthreads();
#pragma unroll
        for (int k = 0; k * kThreads < G * HD; ++k)
            if (tid + k * kThreads < G * HD) qs[tid + k * kThreads] = qv[k];
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf((float)HD);
    const int passes = (nv + P - 1) / P;
#pragma unroll 2
    for (int ps = 0; ps < passes; ++ps) {
        const int pi = ps * P + pg;
        const bool valid = pi < nv;
        float dot[G];
#pragma unroll
        for (int j = 0; j < G; ++j) dot[j] = 0.f;
        if (valid) {
            float kf[8];
            ld8<KT>((const KT *)(k_lds + (size_t)pi * Geo::ROW) + d8 * 8, kf);
#pragma unroll
            for (int j = 0; j < G; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) dot[j] = fmaf(kf[e], qs[j * HD + d8 * 8 + e], dot[j]);
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float s = group_sum<T>(dot[j]);
            if (d8 == 0 && valid) sh.p[pi][j] = s * scale;
        }
    }
    __syncthreads();
    mark(1);
    for (int j = wave; j < G; j += kWaves) {
        float mx = -INFINITY;
        for (int c = lane; c < nv; c += 64) mx = fmaxf(mx, sh.p[c][j]);
        mx = wave_max(mx);
        float sum = 0.f;
        for (int c = lane; c < nv; c += 64) {
            const float pv = expf(sh.p[c][j] - mx);
            sh.p[c][j] = pv;
            sum += pv;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            sh.m[j] = mx;
            sh.l[j] = sum;
        }
    }
    __syncthreads();
    mark(2);
    // Weighted V: lane owns DPL head dimensions, wave w positions w, w + 4,
    // ...; the four waves' sums are added in wave order.
    constexpr int DPL = HD / 64;
    float acc[G][DPL];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
#pragma unroll 4
    for (int pi = wave; pi < nv; pi += kWaves) {
        const KT *vrow = (const KT *)(v_lds + (size_t)pi * Geo::ROW) + lane * DPL;
        float vf[DPL];
        if constexpr (sizeof(KT) == 2) {
            if constexpr (DPL == 1) {
                vf[0] = bf16_f32(*vrow);
            } else {
                const uint32_t w2 = *(const uint32_t *)vrow;
                vf[0] = bf16_lo(w2);
                vf[1] = bf16_hi(w2);
            }
        } else {
#pragma unroll
            for (int e = 0; e < DPL; ++e) vf[e] = vrow[e];
        }
        float pj[AttnShm<HD, G, CH>::GP];
#pragma unroll
        for (int j4 = 0; j4 < AttnShm<HD, G, CH>::GP; j4 += 4) {
            const f32x4 q4 = *(const f32x4 *)&sh.p[pi][j4];
            pj[j4] = q4[0];
            pj[j4 + 1] = q4[1];
            pj[j4 + 2] = q4[2];
            pj[j4 + 3] = q4[3];
        }
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[j][e] = fmaf(pj[j], vf[e], acc[j][e]);
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < DPL; ++e) sh.red[wave][j][lane * DPL + e] = acc[j][e];
    __syncthreads();
    mark(3);
    // Partials of group g, split-major: [split][head of group][HD + 2].
    uint64_t *gpart = a.part + (size_t)g * a.max_splits * G * (HD + 2);
    uint64_t *part = gpart + (size_t)split * G * (HD + 2);
    for (int t = tid; t < G * HD; t += kThreads) {
        const int j = t / HD, d = t % HD;
        float o = sh.red[0][j][d];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) o += sh.red[w][j][d];
        stf(part + (size_t)j * (HD + 2) + d, o, tB);
    }
    if (tid < G) {
        stf(part + (size_t)tid * (HD + 2) + HD, sh.m[tid], tB);
        stf(part + (size_t)tid * (HD + 2) + HD + 1, sh.l[tid], tB);
    }
    if (split != 0) return true;
    // The split-0 item merges the group's S partials in split order
    // (weights exp(m_s - M), sum L = sum_s w_s l_s) and publishes the
    // group's attention output.
    if (!gather_lds(tb, gpart, S * G * (HD + 2), tB, a.abort_flag)) return false;
    if (tid < G) {
        float M = -INFINITY;
        for (int s = 0; s < S; ++s) M = fmaxf(M, val_of(tb[((size_t)s * G + tid) * (HD + 2) + HD]));
        float L = 0.f;
        for (int s = 0; s < S; ++s) {
            const uint64_t *ps = tb + ((size_t)s * G + tid) * (HD + 2);
            const float w = expf(val_of(ps[HD]) - M);
            sh.p[s][tid] = w;
            L = fmaf(w, val_of(ps[HD + 1]), L);
        }
        sh.l[tid] = 1.0f / L;
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += kThreads) {
        const int j = t / HD, d = t % HD;
        float o = 0.f;
        for (int s = 0; s < S; ++s) o = fmaf(sh.p[s][j], val_of(tb[((size_t)s * G + j) * (HD + 2) + d]), o);
        stf(a.attn + (size_t)(g * G + j) * HD + d, o * sh.l[j], tB);
    }
    return true;
}

// LM head rows gw, gw + W, ... of one wave against the final-normed hidden
// state xs: logits, and the wave's best (key, index). Out of line, so that
// its double-buffered rows are register-allocated apart from the layer loop.
template <int UHB>
__device__ __noinline__ void head_dots(const uint16_t *head, float *logits, const float *xs, int H, int V, int gw,
                                       int W, int head_rows, int &key, uint32_t &idx) {
    constexpr int HB = 4;  // rows per batch, two batches in flight
    const int lane = tid_here() & 63, nHB = H / 8;
    const size_t stride = (size_t)H * 2;
    u32x4 hb[2][HB][UHB];
    const int nbat = (head_rows + HB - 1) / HB;
    auto issue = [&](u32x4 (&buf)[HB][UHB], int bi) {
#pragma unroll
        for (int k = 0; k < HB; ++k) {
            const int i = bi * HB + k;
            if (i < head_rows) load_row(buf[k], (const uint8_t *)head + (size_t)(gw + W * i) * stride, nHB);
        }
    };
    auto consume = [&](const u32x4 (&buf)[HB][UHB], int bi) {
        const int nr = min(HB, head_rows - bi * HB);
        float y[HB];
        dot_rows<FMT_BF16>(buf, xs, nHB, nr, y);
#pragma unroll
        for (int k = 0; k < HB; ++k)
            if (k < nr) {
                const uint32_t r = (uint32_t)(gw + W * (bi * HB + k));
                if (lane == 0) logits[r] = y[k];
                better(key, idx, total_key(y[k]), r);
            }
    };
    issue(hb[0], 0);
    for (int bi = 0; bi < nbat; bi += 2) {
        if (bi + 1 < nbat) issue(hb[1], bi + 1);
        consume(hb[0], bi);
        if (bi + 2 < nbat) issue(hb[0], bi + 2);
        if (bi + 1 < nbat) consume(hb[1], bi + 1);
    }
}

// UH/UQ/UI: 16-byte units per lane of a row with H / q_heads*HD / I
// columns; RGU: gate/up rows per wave; UHB: units per lane of a BF16 head row.
template <int FMT, int HD, int G, class KT, int UH, int UQ, int UI, int RGU, int UHB>
__global__ __launch_bounds__(kThreads) void decode_flow_kernel(FusedArgs a) {
    using Geo = AttnGeo<HD, KT>;
    using U = Unit<FMT, 16>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ Shm sm;
    __shared__ AttnShm<HD, G, Geo::CH> ash;
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    const int NB = gridDim.x, W = NB * kWaves, b = blockIdx.x;
    const int gw0 = b * kWaves + wave;
    const int H = a.H, I = a.I, V = a.V;
    const int qd = a.q_heads * HD, kvd = a.kv_heads * HD;
    const int nH = H / U::E, nQ = qd / U::E, nI = I / U::E;
    const int npairs = (qd + 2 * kvd) / 2;
    const int half = a.rotary / 2;
    const LdsLayout lay = lds_layout(H, I, a.q_heads, HD, G, (int)sizeof(KT), NB, a.max_splits);
    uint64_t *tb = (uint64_t *)lds;
    float *xs = (float *)(lds + lay.xs);

    const bool hasA = b * kWaves < npairs, myA = gw0 < npairs;
    const bool hasH = b * kWaves < H, myH = gw0 < H;
    // Gate/up rows: block b owns RB consecutive rows, wave w rows w, w + 8, ...
    const int RB = (I + NB - 1) / NB;
    const bool hasD = b * RB < I;
    const int head_rows = gw0 < V ? (V - 1 - gw0) / W + 1 : 0;
    const bool hasHead = b * kWaves < V;
    // Blocks that own head rows write argmax partials. Blocks without would
    // have nothing pacing them and could overwrite a step's partials before
    // they are read, so they write none.
    const int head_blocks = min(NB, (V + kWaves - 1) / kWaves);

    int token = __hip_atomic_load(a.step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    long pos = __hip_atomic_load(a.step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float h_own = 0.f;

    u32x4 wA[2][UH], wC[1][UQ], wD[2 * RGU][UH], wE[1][UI];

    // QKV rows of layer l: issued one phase early (before the previous
    // layer's down-phase wait, or before the argmax wait for layer 0).
    auto load_wA = [&](int l) {
        if (myA) {
            const FusedLayer ly = load_layer(a.layers, l);
            const int gw = gw_here();
            load_row(wA[0], ly.qkv + (size_t)(2 * gw) * a.qkv_stride, nH);
            load_row(wA[1], ly.qkv + (size_t)(2 * gw + 1) * a.qkv_stride, nH);
        }
    };
    load_wA(0);

    const int PH = fused_phases_per_step(a.L);
    // A block is paced when it waited on the previous step's last layer (or
    // this is the launch's first step): only then are the cached K/V rows of
    // every earlier position written when it starts a step. Blocks with no
    // role in the previous step may run ahead and must not prefetch them.
    const bool always_paced = hasA || hasH || hasD || hasHead;
    bool item_prev = false;
    for (int s = 0; s < a.steps; ++s, ++pos) {
        // Optional per-phase timestamps of one step (thread 0 of each block).
        const bool traced = a.trace && s == a.trace_step;
        auto mark = [&](int ev) {
            if (traced && tid == 0) a.trace[(size_t)b * (16 * a.L + 3) + ev] = wall_clock64();
        };
        const unsigned tb0 = a.tag0 + (unsigned)(s * PH);
        const long ctx = pos + 1;
        const int S = (int)((ctx + Geo::CH - 1) / Geo::CH);
        const int it = NB - 1 - b;
        const bool hasB = it < a.kv_heads * S;
        const int ig = hasB ? it / S : 0, isplit = hasB ? it % S : 0;
        const bool paced = s == 0 || always_paced || item_prev;
        item_prev = hasB;
        const float *cr = a.rope_cos + (size_t)pos * half;
        const float *sr = a.rope_sin + (size_t)pos * half;
        const int page = a.page_table[pos / TP];
        const int slot = (int)(pos % TP);
        const uint16_t *emb = a.embed + (size_t)token * H;

        for (int l = 0; l < a.L; ++l) {
            const FusedLayer ly = load_layer(a.layers, l);
            const int gw = gw_here();
            const unsigned tA = tb0 + 5 * l, tB = tA + 1, tC = tA + 2, tD = tA + 3, tE = tA + 4;
            const long kv_start = (long)isplit * Geo::CH, kv_lim = min(kv_start + Geo::CH, pos);
            // Weight rows of the o and gate/up phases go out right after the
            // QKV phase (attention blocks: gate/up before attention, o after
            // it), so they stream while attention runs; down rows go out
            // before the down phase's input wait.
            auto load_wD = [&]() {
#pragma unroll
                for (int k = 0; k < RGU; ++k) {
                    const int j = (gw - b * kWaves) + kWaves * k, r = b * RB + j;
                    if (j < RB && r < I) {
                        load_row(wD[2 * k], ly.gate + (size_t)r * a.gu_stride, nH);
                        load_row(wD[2 * k + 1], ly.up + (size_t)r * a.gu_stride, nH);
                    }
                }
            };
            auto load_wC = [&]() {
                if (myH) load_row(wC[0], ly.o + (size_t)gw * a.o_stride, nQ);
            };
            mark(16 * l);

            // ---- A: QKV pairs + RoPE + K/V append. Attention blocks without
            // QKV rows start loading their cached K/V rows now.
            const bool kv_early = hasB && !hasA && (l > 0 || paced);
            if (kv_early) {
                uint8_t *k_lds = (uint8_t *)(tb + lay.qkw);
                load_kv_lds<HD, KT>(k_lds, k_lds + Geo::CH * Geo::ROW, a, ly, ig, kv_start, kv_lim);
            }
            if (hasB) load_wD();
            if (hasA) {
                if (l == 0) {
                    stage_embed(xs, emb, H, ly.ln1, a.eps, sm.red);
                } else {
                    if (!gather_lds(tb, a.hid1, H, tA - 1, a.abort_flag)) return;
                    stage_lds(xs, tb, H, ly.ln1, a.eps, sm.red);
                }
            }
            mark(16 * l + 1);
            if (myA) {
                const int r0 = 2 * gw;
                float y[2];
                dot_rows<FMT>(wA, xs, nH, 2, y);
                float v0 = y[0], v1 = y[1];
                if (lane == 0) {
                    if (ly.qkv_sc) {
                        v0 = v0 * ly.qkv_sc[r0];
                        v1 = v1 * ly.qkv_sc[r0 + 1];
                    }
                    if (ly.qkv_bias) {
                        v0 = v0 + ly.qkv_bias[r0];
                        v1 = v1 + ly.qkv_bias[r0 + 1];
                    }
                    int i0, i1, c0 = -1, c1 = -1;  // q/K/V word, cache element
                    if (r0 < qd + kvd) {
                        const bool is_q = r0 < qd;
                        const int base = is_q ? r0 : r0 - qd;
                        const int h = base / HD, d0 = base % HD;
                        int o0 = d0, o1 = d0 + 1;
                        if (d0 < a.rotary) {
                            const int i = d0 / 2;
                            const float c = cr[i], sn = sr[i];
                            const float x1 = v0 * c - v1 * sn, x2 = v1 * c + v0 * sn;
                            v0 = x1;
                            v1 = x2;
                            o0 = i;
                            o1 = half + i;
                        }
                        if (is_q) {
                            const int q0 = (h / G) * (G + 2) * HD + (h % G) * HD;
                            i0 = q0 + o0;
                            i1 = q0 + o1;
                        } else {
                            const int k0 = h * (G + 2) * HD + G * HD;
                            i0 = k0 + o0;
                            i1 = k0 + o1;
                            const int e0 = ((page * a.kv_heads + h) * TP + slot) * HD;
                            c0 = e0 + o0;
                            c1 = e0 + o1;
                        }
                    } else {
                        const int base = r0 - qd - kvd;
                        const int h = base / HD, d0 = base % HD;
                        const int v0i = h * (G + 2) * HD + (G + 1) * HD;
                        i0 = v0i + d0;
                        i1 = v0i + d0 + 1;
                        const int e0 = ((page * a.kv_heads + h) * TP + slot) * HD;
                        c0 = (e0 + d0) | (1 << 30);
                        c1 = (e0 + d0 + 1) | (1 << 30);
                    }
                    sm.outv[2 * wave] = v0;
                    sm.outv[2 * wave + 1] = v1;
                    sm.outi[2 * wave] = i0;
                    sm.outi[2 * wave + 1] = i1;
                    sm.outc[2 * wave] = c0;
                    sm.outc[2 * wave + 1] = c1;
                }
            }
            if (hasA) {
                // The block's pairs leave as one run: q/K/V words (K/V as
                // the cache holds them) and the K/V cache elements.
                __syncthreads();
                const int n = 2 * min(kWaves, npairs - b * kWaves);
                if (tid < n) {
                    const float v = sm.outv[tid];
                    const int c = sm.outc[tid];
                    if (c >= 0) {
                        KT *cache = (KT *)((c >> 30) ? ly.vc : ly.kc);
                        st_kv(cache + (c & ((1 << 30) - 1)), v);
                    }
                    stf(a.qkvn + sm.outi[tid], c >= 0 ? kv_round<KT>(v) : v, tA);
                }
            }
            mark(16 * l + 2);
            if (!hasB) {
                load_wC();
                load_wD();
            }

            // ---- B: attention item.
            if (hasB) {
                if (hasA) {
                    uint8_t *k_lds = (uint8_t *)(tb + lay.qkw);
                    load_kv_lds<HD, KT>(k_lds, k_lds + Geo::CH * Geo::ROW, a, ly, ig, kv_start, kv_lim);
                }
                uint64_t *tr = traced ? a.trace + (size_t)b * (16 * a.L + 3) + 16 * l + 3 : nullptr;
                if (!attn_item<HD, G, KT>(a, ly, tb, ig, isplit, S, pos, tA, tB, !hasA && !kv_early, lay.qkw, ash, tr))
                    return;
                load_wC();
            }
            mark(16 * l + 7);

            // ---- C: merge + o_proj + residual.
            if (hasH) {
                if (!gather_lds(tb, a.attn, qd, tB, a.abort_flag)) return;
                stage_lds(xs, tb, qd, nullptr, 0.f, sm.red);
            }
            mark(16 * l + 8);
            if (myH) {
                float y[1];
                dot_rows<FMT>(wC, xs, nQ, 1, y);
                float v = y[0];
                if (ly.o_sc) v = v * ly.o_sc[gw];
                if (ly.o_bias) v = v + ly.o_bias[gw];
                const float old = l == 0 ? bf16_f32(emb[gw]) : h_own;
                h_own = old + v;
                if (lane == 0) sm.outv[wave] = h_own;
            }
            if (hasH) publish(a.hid0 + b * kWaves, sm.outv, min(kWaves, H - b * kWaves), tC);
            mark(16 * l + 9);

            // ---- D: gate/up + SwiGLU.
            if (hasD) {
                if (!gather_lds(tb, a.hid0, H, tC, a.abort_flag)) return;
                stage_lds(xs, tb, H, ly.ln2, a.eps, sm.red);
            }
            mark(16 * l + 10);
            if (myH) load_row(wE[0], ly.down + (size_t)gw * a.down_stride, nI);
            {
                int nr = 0;
#pragma unroll
                for (int k = 0; k < RGU; ++k) {
                    const int j = wave + kWaves * k;
                    nr += j < RB && b * RB + j < I ? 2 : 0;
                }
                float y[2 * RGU];
                dot_rows<FMT>(wD, xs, nH, nr, y);
#pragma unroll
                for (int k = 0; k < RGU; ++k) {
                    const int j = wave + kWaves * k, r = b * RB + j;
                    if (j < RB && r < I) {
                        float gv = y[2 * k], uv = y[2 * k + 1];
                        if (ly.gate_sc) {
                            gv = gv * ly.gate_sc[r];
                            uv = uv * ly.up_sc[r];
                        }
                        if (lane == 0) sm.outv[j] = gv * (uv / (1.0f + expf(-gv)));
                    }
                }
            }
            if (hasD) publish(a.act + b * RB, sm.outv, min(RB, I - b * RB), tD);
            mark(16 * l + 11);

            // ---- E: down + residual.
            if (l + 1 < a.L) load_wA(l + 1);
            if (hasH) {
                if (!gather_lds(tb, a.act, I, tD, a.abort_flag)) return;
                stage_lds(xs, tb, I, nullptr, 0.f, sm.red);
            }
            mark(16 * l + 12);
            if (myH) {
                float y[1];
                dot_rows<FMT>(wE, xs, nI, 1, y);
                float v = y[0];
                if (ly.down_sc) v = v * ly.down_sc[gw];
                h_own = h_own + v;
                if (lane == 0) sm.outv[wave] = h_own;
            }
            if (hasH) publish(a.hid1 + b * kWaves, sm.outv, min(kWaves, H - b * kWaves), tE);
            mark(16 * l + 13);
        }

        // ---- LM head (BF16, final norm fused) + argmax partials.
        const unsigned tH = tb0 + 5 * a.L;
        int key = INT_MIN;
        uint32_t idx = 0;
        if (hasHead) {
            if (!gather_lds(tb, a.hid1, H, tH - 1, a.abort_flag)) return;
            stage_lds(xs, tb, H, a.final_norm, a.eps, sm.red);
            mark(16 * a.L);
            head_dots<UHB>(a.head, a.logits, xs, H, V, gw_here(), W, head_rows, key, idx);
        }
        block_best(key, idx, sm);
        mark(16 * a.L + 1);
        uint64_t *am = a.am + (size_t)(s & 1) * NB * 2;
        if (hasHead && tid == 0) {
            stt(am + 2 * b, (uint32_t)key, tH);
            stt(am + 2 * b + 1, idx, tH);
        }
        if (s + 1 < a.steps) load_wA(0);
        // Blocks that use the token (embedding row, residual) reduce the
        // partials of every head block.
        if (hasA || hasH) {
            if (!gather_lds(tb, am, 2 * head_blocks, tH, a.abort_flag)) return;
            key = INT_MIN;
            idx = 0;
            for (int i = tid; i < head_blocks; i += kThreads)
                better(key, idx, (int)(uint32_t)tb[2 * i], (uint32_t)tb[2 * i + 1]);
            block_best(key, idx, sm);
            token = (int)idx;
            if (b == 0 && tid == 0) {
                if (pos + 1 < a.hist_cap)
                    __hip_atomic_store(a.hist + pos + 1, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store((uint32_t *)a.step, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(a.step + 1, (int32_t)(pos + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        mark(16 * a.L + 2);
    }
}

struct Variant {
    int fmt, hd, g, uh, uq, ui, rgu, uhb;
};

// Shapes with a built kernel: Qwen2-0.5B (hidden 896, 14/2 heads of 64,
// intermediate 4864) and the two small test shapes.
constexpr Variant kVariants[] = {
    {FMT_BF16, 64, 7, 2, 2, 10, 3, 2},
    {FMT_BF16, 64, 2, 1, 1, 1, 1, 1},
    {FMT_BF16, 128, 4, 1, 2, 2, 1, 1},
};

int units_per_lane(int cols, int elems_per_unit) { return (cols / elems_per_unit + 63) / 64; }

const Variant *find_variant(int fmt, int H, int q_heads, int kv_heads, int hd, int I, int blocks) {
    if (kv_heads <= 0 || q_heads % kv_heads) return nullptr;
    const int g = q_heads / kv_heads, E = fmt == FMT_Q8 ? 16 : 8, W = blocks * kWaves;
    const int qd = q_heads * hd, kvd = kv_heads * hd;
    if (H % 8 || qd % E || H % E || I % E) return nullptr;
    if ((qd + 2 * kvd) / 2 > W || H > W) return nullptr;
    for (const Variant &v : kVariants) {
        if (v.fmt != fmt || v.hd != hd || v.g != g) continue;
        if (units_per_lane(H, E) > v.uh || units_per_lane(qd, E) > v.uq || units_per_lane(I, E) > v.ui) continue;
        const int rb = (I + blocks - 1) / blocks;
        if (rb > kStage || (rb + kWaves - 1) / kWaves > v.rgu || units_per_lane(H, 8) > v.uhb) continue;
        return &v;
    }
    return nullptr;
}

template <int FMT, int HD, int G, class KT, int UH, int UQ, int UI, int RGU, int UHB>
int launch_one(const FusedArgs &a, int nb, hipStream_t s) {
    auto k = decode_flow_kernel<FMT, HD, G, KT, UH, UQ, UI, RGU, UHB>;
    const size_t lds = (size_t)lds_layout(a.H, a.I, a.q_heads, HD, G, (int)sizeof(KT), nb, a.max_splits).total;
    hipFuncAttributes attr{};
    CHIP_CHECK(hipFuncGetAttributes(&attr, (const void *)k));
    if (attr.sharedSizeBytes + lds > device_max_lds())
        return fail("HIP backend: persistent decode needs more LDS than a block has.");
    void *args[] = {(void *)&a};
    CHIP_CHECK(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    // CHEETAH_HIP_FUSED_PLAIN_LAUNCH=1: an ordinary launch instead of the
    // cooperative one (for tools that do not handle cooperative launches).
    // One block per CU is co-resident on an otherwise idle device; were it
    // not, the bounded polls time out and the call fails.
    const char *plain = getenv("CHEETAH_HIP_FUSED_PLAIN_LAUNCH");
    if (plain && plain[0] == '1')
        CHIP_CHECK(hipLaunchKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s));
    else
        CHIP_CHECK(hipLaunchCooperativeKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s));
    return 0;
}

template <class KT>
int launch_kt(const Variant &v, const FusedArgs &a, int nb, hipStream_t s) {
    if (v.hd == 64 && v.g == 7) return launch_one<FMT_BF16, 64, 7, KT, 2, 2, 10, 3, 2>(a, nb, s);
    if (v.hd == 64 && v.g == 2) return launch_one<FMT_BF16, 64, 2, KT, 1, 1, 1, 1, 1>(a, nb, s);
    if (v.hd == 128 && v.g == 4) return launch_one<FMT_BF16, 128, 4, KT, 1, 2, 2, 1, 1>(a, nb, s);
    return fail("HIP backend: no persistent decode kernel for this shape.");
}

}  // namespace

int fused_positions_per_item(int head_dim, bool kv_f32) {
    (void)head_dim;
    (void)kv_f32;
    return TP;
}

bool fused_decode_supported(int fmt, int H, int q_heads, int kv_heads, int head_dim, int I, bool aligned16,
                            int blocks) {
    return aligned16 && blocks > 0 && find_variant(fmt, H, q_heads, kv_heads, head_dim, I, blocks) != nullptr;
}

int fused_decode_blocks() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

int fused_max_splits(int H, int q_heads, int kv_heads, int head_dim, int I, bool kv_f32, int blocks,
                     size_t capacity) {
    // Splits whose partials fit the LDS budget next to everything else.
    const int kvb = kv_f32 ? 4 : 2;
    const LdsLayout base = lds_layout(H, I, q_heads, head_dim, q_heads / kv_heads, kvb, blocks, 1);
    const int G = q_heads / kv_heads;
    const int spare_words = (kLdsBudget - (base.total - base.tbw * 8)) / 8 - kChunk - 2;
    const int fit = std::min(spare_words / (G * (head_dim + 2)), TP);  // merge weights fill one LDS row per split
    const size_t per_item = (size_t)fused_positions_per_item(head_dim, kv_f32);
    const size_t need = (capacity + per_item - 1) / per_item;
    int ms = blocks / kv_heads;
    ms = std::min(ms, fit);
    ms = (int)std::min((size_t)ms, need);
    return std::max(ms, 1);
}

int launch_decode_fused(const FusedArgs &a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s) {
    const int nb = fused_decode_blocks();
    if (nb <= 0) return fail("HIP backend: cannot size the persistent decode grid.");
    const Variant *v = find_variant(fmt, a.H, a.q_heads, a.kv_heads, head_dim, a.I, nb);
    if (!v || v->g != group) return fail("HIP backend: no persistent decode kernel for this shape.");
    return kv_f32 ? launch_kt<float>(*v, a, nb, s) : launch_kt<uint16_t>(*v, a, nb, s);
}

}  // namespace chip
