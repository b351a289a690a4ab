// Persistent dataflow decode kernel: one cooperative launch (one 512-thread
// block per CU) runs whole decode steps -- embedding, every layer, LM head,
// greedy argmax -- with no device-wide barrier.
//
// The grid is split into fixed roles (FusedGeom):
//   items  one q head over one run of positions: its 64 q rows (fused
//          RMSNorm, bias, RoPE), attention over the run's cached K/V rows
//          (and the new position's, for the run that holds it), and the
//          head's o_proj columns applied to the unnormalised output: an
//          o_proj partial of every hidden row, with the run's max and sum
//   KV     the new position's K and V rows (fused RMSNorm, bias, RoPE),
//          appended to the pages and handed to the items that need them
//   FFN    gate/up rows, SwiGLU and the matching down_proj columns (a down
//          partial of every hidden row); the first of them also own 8
//          residual rows each (one per wave, held in a register)
// Per layer four hand-offs are on the critical path:
//   residual -> items, KV          (the KV -> item hand-off overlaps the
//                                   items' scores of their cached rows)
//   item partials -> owners        owners merge the runs of every head in
//                                  split order (weights exp(m_s - M) / sum)
//                                  and add the residual
//   residual -> FFN blocks
//   down partials -> owners        summed in block order, + residual
// and once per step the LM head (fused final RMSNorm) + per-block argmax
// partials, which the blocks that need the next token reduce themselves
// (ties to the last index, engine.rs:2247-2253).
//
// Every value one block hands to another is a 64-bit word {f32 bits, tag},
// where the tag names the phase instance that produced it (launch base +
// step * (5L + 1) + 5 * layer + phase). Aligned 8-byte stores are
// single-copy atomic, so value and tag arrive together, and a consumer knows
// its inputs are complete when every word it copied carries the expected
// tag.
//
// Weight streaming. Every thread holds a pool of 16-byte weight units in
// registers: an item's q rows and o_proj columns, a KV block's rows, an FFN
// block's gate/up rows and down columns. All blocks refill the pool at one
// point of each layer (after the items' work): items and KV blocks with the
// next layer's rows, FFN blocks with this layer's, so every transfer
// overlaps the hand-offs before its use. Every wave issues the same number
// of loads there whatever its role (units it does not need point past the
// buffer's range and read nothing), so no path through the loop has a
// different load count and the compiler's waits stay exact. The LDS copies
// and the hand-off stores are inline assembly so that the compiler does not
// make LDS reads and later loads wait for them.
//
// Buffer reuse needs no barrier: a block polls a phase's inputs only in a
// phase where it also produces outputs, and every buffer is rewritten only
// by a phase that transitively depends on all of those outputs. Argmax
// partials alternate between two buffers by step parity.
//
// Every poll is bounded: on timeout a block raises the abort word, which all
// polls watch, so every later poll gives up within a few rounds and the
// launch runs to its end on stale values. The host sees the word, discards
// the steps and resets the tagged words. The only data-dependent address,
// the token, keeps its last good value when its poll gives up.
//
// Math per phase is that of the multi-kernel path (gemv.hip, attention.hip,
// misc.hip), i.e. the reference path of ops.rs / qwen2.rs; only f32
// summation orders differ (o_proj is applied per head before the split
// merge, which is linear).
#include <cstdlib>

#include "decode_fused.hpp"
#include "wunit.hpp"

namespace chip {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kDmaWave = kWaves - 1;   // issues the block's copies into LDS
constexpr int TP = 64;                 // positions per KV page
constexpr int kOwn = kWaves;           // residual rows per owner block, one per wave
constexpr int kMaxSplits = 16;         // attention splits per q head, at most
constexpr int kIpMax = 4 * TP;         // positions per attention item, at most
constexpr int kKvLdsMax = 64 * 1024;   // LDS for one item's K and V rows, at most
constexpr int kChunk = 128;            // tagged words per wave-wide 16-byte-per-lane load
constexpr int kXcds = 8;               // the dispatcher places block b on XCD b % 8 (each XCD has its own L2)

// Blocks per attention split: q heads rounded up to the XCD count. Item
// (split s, head h) sits at block s * heads_padded + slot(h), on XCD
// slot(h) % 8 for every s: the splits of one head, which read the same q
// rows and o_proj columns, share one L2, and (fused_item_slots) the heads of
// one KV group, which read the same K/V rows, share a set of XCDs.
__host__ __device__ constexpr int heads_padded(int q_heads) { return (q_heads + kXcds - 1) / kXcds * kXcds; }
constexpr long kSpinLimit = 1L << 20;
constexpr uint32_t kNoRead = 0x80000000u;  // buffer offset past every range

// The f32 vector the dot products read sits in LDS with every 8 elements
// padded to 10 floats: a lane reads the 8 x values of its 16-byte weight unit
// at a 40-byte stride, so the lanes of a quarter wave hit distinct banks (at
// the unpadded 32-byte stride, lanes 8 apart share banks and seven waves
// reading one vector serialise on the conflicts).
__host__ __device__ constexpr int xpad(int i) { return (i >> 3) * 10 + (i & 7); }

// Row stride (elements) of a split vector of k (a multiple of 8) elements
// per part: 16 bytes past the row, so that the four rows start four LDS
// banks apart. The A operand's lanes 0..15 read rows 0, 1, 2, 3, 3, ...
// at the same column; at a stride of a multiple of 128 bytes every row
// would start on the same bank and each read would serialise four ways.
__host__ __device__ constexpr int split_stride(int k) { return k + 8; }

// threadIdx.x through an opaque copy: address arithmetic stays next to its
// use inside the step loop instead of being hoisted out of it and held in
// registers for the whole kernel.
__device__ __forceinline__ int tid_here() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int lane_here() { return tid_here() & 63; }

// Global stores are written as inline assembly (the instructions the
// compiler emits for device-scope relaxed atomic stores: sc1). Vector memory
// loads complete in issue order but stores need not, and the compiler, seeing
// both kinds outstanding, would make every wait for a weight row a wait for
// everything; with stores out of its sight it waits for a row only until the
// loads issued after that row remain, which in-order loads make exact.
__device__ __forceinline__ void st_u64(uint64_t *p, uint64_t v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_u32(void *p, uint32_t v) {
    asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st_u16(void *p, uint32_t v) {
    asm volatile("global_store_short %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void stt(uint64_t *p, uint32_t bits, unsigned tag) { st_u64(p, ((uint64_t)tag << 32) | bits); }
// Two tagged words {a, tag}, {b, tag} at p (16-byte aligned) in one store.
// A vector memory store of more than 64 data bits reads its data registers
// after issue; on this chip a VALU write to them needs two wait states
// after the store, which the compiler inserts for its own stores but cannot
// for one inside inline assembly (it reuses the registers at once). The
// s_nop 1 provides them.
__device__ __forceinline__ void stf2(uint64_t *p, float a, float b, unsigned tag) {
    const u32x4 v = {__float_as_uint(a), tag, __float_as_uint(b), tag};
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void stf(uint64_t *p, float v, unsigned tag) { stt(p, __float_as_uint(v), tag); }
__device__ __forceinline__ float val_of(uint64_t w) { return __uint_as_float((uint32_t)w); }

__device__ __forceinline__ void st_kv(uint16_t *p, float v) { st_u16(p, f32_bf16_rne(v)); }
__device__ __forceinline__ void st_kv(float *p, float v) { st_u32(p, __float_as_uint(v)); }
// The value a K/V element has once stored in the cache.
template <class KT>
__device__ __forceinline__ float kv_round(float v) {
    if constexpr (sizeof(KT) == 2) return bf16_f32(f32_bf16_rne(v));
    else return v;
}

__device__ __forceinline__ bool aborted(const int *f) {
    return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void raise_abort(int *f) { st_u32(f, 1u); }

// Read-only values at a wave-uniform index through the constant address
// space: scalar loads (counted apart from the vector loads of the weights).
template <class T>
__device__ __forceinline__ T ldc(const T *p, long i) {
    return ((const __attribute__((address_space(4))) T *)p)[i];
}
__device__ __forceinline__ float ldc_bf16(const uint16_t *p, long i) {
    const uint32_t w = ldc((const uint32_t *)p, i >> 1);
    return (i & 1) ? bf16_hi(w) : bf16_lo(w);
}

typedef const __attribute__((address_space(4))) FusedArgs CArgs;
typedef const __attribute__((address_space(4))) FusedLayer CLayer;

// The launch's arguments are read where used, through an opaque copy of the
// pointer to them, so that fields are re-read (scalar-cache hits) instead of
// each being held in a scalar register for the whole launch. The pointer is
// taken once, in the kernel's own body (the kernarg-segment intrinsic means
// something only there: in any other function the compiler lowers it to a
// null pointer), and every helper that reads an argument receives it as a
// parameter, so that an outlined helper still reads the right memory.
__device__ __forceinline__ CArgs *opaque(CArgs *a) {
    auto p = (const __attribute__((address_space(4))) char *)a;
    asm volatile("" : "+s"(p));
    return (CArgs *)p;
}
// Layer l's pointer table, read the same way.
__device__ __forceinline__ CLayer *layer_of(CArgs *a, int l) { return (CLayer *)opaque(a)->layers + l; }

// LDS barrier that waits on LDS (and scalar) traffic only: outstanding
// vector memory loads stay in flight across it.
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (lds the same in every lane), device-coherent (sc1). The low 32 bits of a
// generic pointer into LDS are the LDS byte address. The copy takes its LDS
// base from m0, a register the compiler reserves (an asm clobber list cannot
// claim it), so the block saves m0 into a scalar temporary and restores it
// after the copy has issued: whatever value compiler-generated code keeps in
// m0 survives. (The compiler's own global_load_lds builtin would manage m0,
// but it makes every later LDS read wait for all vector loads in flight,
// weight rows included.)
__device__ __forceinline__ void dma16(const void *g, const void *lds) {
    const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off sc1\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(l)
        : "memory");
}
// dma16 without the coherence bit, for data no block writes while it is
// read (embedding and gain rows; K/V rows of positions already written,
// which no later write touches): L2 hits across the blocks of one XCD.
__device__ __forceinline__ void dma16_nc(const void *g, const void *lds) {
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
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// N (1 or 2) device-coherent 16-byte loads p[i] -> r[i] and the wait for
// all of them in one asm statement: no instruction sees r before its load
// has landed.
template <int N>
__device__ __forceinline__ void poll16(u32x4 (&r)[2], const uint64_t *const (&p)[2]) {
    static_assert(N == 1 || N == 2, "one or two chunks per wave");
    if constexpr (N == 1)
        asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0])
                     : "v"(p[0])
                     : "memory");
    else
        asm volatile("global_load_dwordx4 %0, %2, off sc1\n\tglobal_load_dwordx4 %1, %3, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1])
                     : "v"(p[0]), "v"(p[1])
                     : "memory");
}

// Both words of a 16-byte unit (value, tag, value, tag) at word w of n carry
// `tag` (words past n count as fresh).
__device__ __forceinline__ bool unit_fresh(u32x4 v, int w, int n, unsigned tag) {
    return (w >= n || v[1] == tag) && (w + 1 >= n || v[3] == tag);
}

// A gather's source: tagged words A[0, nA) in 128-word chunks [0, cA) of the
// LDS copy, then B[0, nB) in the chunks after them.
struct Ranges {
    const uint64_t *a, *b;
    int na, nb;
};

// Register form of the gather for a wave that owns N <= 2 chunks (w and
// w + 8): a round loads every chunk of the wave into registers and waits
// for all of them (one asm statement), then checks the tags there; once
// every word is fresh the chunks are written to LDS. Re-loading fresh
// chunks costs traffic but no time: a round takes one memory round trip
// either way.
template <int N>
__device__ __forceinline__ void gather_regs(uint64_t *dst, Ranges g, unsigned tag, int *abort_flag, int wave, int lane) {
    const int ca = (g.na + kChunk - 1) / kChunk;
    const uint64_t *p[2];
    int n[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = wave + kWaves * i;
        const bool in_a = c < ca;
        const int base = (in_a ? c : c - ca) * kChunk;
        n[i] = (in_a ? g.na : g.nb) - base;  // valid words of the chunk
        const uint64_t *src = in_a ? g.a : g.b;
        p[i] = i < N && lane * 2 < n[i] ? src + base + lane * 2 : g.a;
    }
    long spins = 0;
    while (true) {
        u32x4 r[2];
        poll16<N>(r, p);
        bool stale = false;
#pragma unroll
        for (int i = 0; i < N; ++i) stale |= !unit_fresh(r[i], lane * 2, n[i], tag);
        const bool done = !__any(stale);
        const bool give_up = !done && (++spins > kSpinLimit || ((spins & 15) == 0 && aborted(abort_flag)));
        if (done || give_up) {
            // On a give-up the words are written too, stale or not: they are
            // the source buffer's, so what readers take from them (a token's
            // row index) stays one that buffer held.
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (lane * 2 < n[i]) *(u32x4 *)(dst + (wave + kWaves * i) * kChunk + lane * 2) = r[i];
            if (give_up) raise_abort(abort_flag);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// All waves: copies tagged words into LDS (range A at dst[0, nA), range B
// from the next 128-word boundary on) and waits until each carries `tag`.
// Wave w owns the 128-word chunks w and w + 8 (at most 16 chunks) and polls
// them in registers (gather_regs). The caller's barrier then makes all of
// them visible to the block. A wave's wait also covers the weight rows it
// has in flight. On timeout the abort word is raised and the wave moves on
// with what it has. Inline (no call), so the weight registers held across
// it need no call-preserved registers.
constexpr int kMaxGather = 2 * kWaves * kChunk;
__device__ __forceinline__ void gather(uint64_t *dst, Ranges g, unsigned tag, int *abort_flag) {
    const int lane = lane_here(), wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int chunks = (g.na + kChunk - 1) / kChunk + (g.nb + kChunk - 1) / kChunk;
    if (chunks > wave + kWaves) gather_regs<2>(dst, g, tag, abort_flag, wave, lane);
    else if (chunks > wave) gather_regs<1>(dst, g, tag, abort_flag, wave, lane);
}
__device__ __forceinline__ void gather(uint64_t *dst, const uint64_t *src, int n, unsigned tag, int *abort_flag) {
    gather(dst, Ranges{src, src, n, 0}, tag, abort_flag);
}

// One wave: polls words [base, base + 128) of src (n words in all) into
// registers until every one of them carries `tag` (lane l holds words
// base + 2 l and base + 2 l + 1 as value, tag, value, tag; lanes past n
// hold src[0], counted as fresh). Bounded like gather_regs: on timeout it
// raises the abort word and returns what it loaded.
__device__ __forceinline__ u32x4 poll_chunk(const uint64_t *src, int base, int n, unsigned tag, int *abort_flag) {
    const int lane = lane_here(), cnt = n - base;
    const uint64_t *p[2] = {lane * 2 < cnt ? src + base + lane * 2 : src, src};
    long spins = 0;
    while (true) {
        u32x4 r[2];
        poll16<1>(r, p);
        const bool done = !__any(!unit_fresh(r[0], lane * 2, cnt, tag));
        const bool give_up = !done && (++spins > kSpinLimit || ((spins & 15) == 0 && aborted(abort_flag)));
        if (done || give_up) {
            if (give_up) raise_abort(abort_flag);
            return r[0];
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// One wave: starts copying `bytes` (a multiple of 16) from global memory
// into LDS; completion is awaited with wait_vm.
__device__ __forceinline__ void dma_bytes(void *dst, const void *src, int bytes) {
    const int lane = lane_here();
    for (int c = 0; c < bytes; c += 1024) {
        const int byte = c + lane * 16;
        if (byte < bytes) dma16((const uint8_t *)src + byte, (uint8_t *)dst + c);
    }
}

// One wave: the RMSNorm scale of n values, inv = 1 / sqrt(mean(x^2) +
// eps) (ops.rs:646-652); x the values of the tagged words src or the BF16
// row src.
template <bool BF16_SRC>
__device__ __forceinline__ float wave_norm_scale(const void *src, int n, float eps) {
    const int lane = lane_here();
    float ss = 0.f;
#pragma unroll 4
    for (int i = lane; i < n; i += 64) {
        float v;
        if constexpr (BF16_SRC) v = bf16_f32(((const uint16_t *)src)[i]);
        else v = val_of(((const uint64_t *)src)[i]);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

// All waves: xs[xpad(i)] = x[i], or x[i] * (inv * g[i]) with a BF16 gain row g
// (the GEMV prologue's RMSNorm).
template <bool BF16_SRC>
__device__ __forceinline__ void block_stage(float *xs, const void *src, int n, const uint16_t *g, float inv) {
#pragma unroll 4
    for (int i = tid_here(); i < n; i += kThreads) {
        float v;
        if constexpr (BF16_SRC) v = bf16_f32(((const uint16_t *)src)[i]);
        else v = val_of(((const uint64_t *)src)[i]);
        xs[xpad(i)] = g ? v * (inv * bf16_f32(g[i])) : v;
    }
}

typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const void *base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// Compute waves: one weight row as 16-byte units (unit u in lane u % 64,
// slot u / 64) by buffer loads issued whether or not the row is the wave's:
// lanes without a unit of an owned row read past the range (nothing).
template <int N>
__device__ __forceinline__ void load_row(u32x4 (&w)[N], Rsrc r, uint32_t row_off, int n_units, bool valid) {
    const int lane = lane_here();
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = lane + 64 * k;
        const uint32_t off = valid && u < n_units ? row_off + (uint32_t)u * 16u : kNoRead;
        w[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
    }
}

// Wave-wide dot products of R loaded rows with xs; a unit's x values are
// read once for all rows. Per row the summation order is fixed (unit, then
// element); results land in every lane. Branch-free: lanes past the row
// (n_units) read a valid x at a clamped index while their weights are the
// zeros of a load that read nothing, and rows a wave does not own are
// computed from such zeros too, so every path consumes every loaded
// register (a path that skipped one would make the compiler wait for its
// load before reusing the register).
template <int FMT, int R, int N>
__device__ __forceinline__ void dot_rows(const u32x4 (&w)[R][N], const float *xs, int n_units, float (&out)[R]) {
    using U = Unit<FMT, 16>;
    const int lane = lane_here();
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = min(lane + 64 * k, n_units - 1);
        float xv[U::E];
#pragma unroll
        for (int e = 0; e < U::E; ++e) xv[e] = xs[xpad(u * U::E + e)];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t raw[4] = {w[i][k][0], w[i][k][1], w[i][k][2], w[i][k][3]};
            U::decode(raw, [&](int e, float v) { acc[i] = fmaf(v, xv[e], acc[i]); });
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) out[i] = wave_sum(acc[i]);
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
__device__ __forceinline__ void wave_best(int &key, uint32_t &idx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int k2 = __shfl_xor(key, off, 64);
        const uint32_t i2 = __shfl_xor(idx, off, 64);
        better(key, idx, k2, i2);
    }
}

constexpr int kStage = 64;  // outputs one block publishes per phase, at most

struct Shm {
    int ikey[kWaves];
    uint32_t iidx[kWaves];
    int token;                 // the step's sampled id
    float out[kStage];         // a phase's outputs of the block, stored as one run
    float red[kWaves][128];    // each wave's tile outputs over its input chunk (up to 8 tiles of 16)
    float ss[kWaves];          // each wave's sum of squares of its chunk (polled RMSNorm input)
    alignas(16) uint16_t dp[4][split_stride(32)];  // an FFN block's SwiGLU outputs, split (put_split)
};

// Reduces (key, idx) over the block; the result lands in every thread.
__device__ __forceinline__ void block_best(int &key, uint32_t &idx, Shm &sm) {
    const int lane = lane_here(), wave = tid_here() >> 6;
    wave_best(key, idx);
    if (lane == 0) {
        sm.ikey[wave] = key;
        sm.iidx[wave] = idx;
    }
    bar();
    key = sm.ikey[0];
    idx = sm.iidx[0];
    for (int w = 1; w < kWaves; ++w) better(key, idx, sm.ikey[w], sm.iidx[w]);
    bar();
}


// Keeps loaded rows in their registers across code that would otherwise
// reuse them (the compiler then waits for their loads here).
template <int R, int N>
__device__ __forceinline__ void pin(u32x4 (&w)[R][N]) {
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int k = 0; k < N; ++k) asm volatile("" : "+v"(w[i][k]));
}

// LM head rows gw, gw + W, ... of one wave against the final-normed hidden
// state xs: logits, and the wave's best (key, index). Batches of HB rows, two
// in flight; every batch issues HB rows of loads (rows past head_rows read
// nothing), so the waits count exactly. Measured on the Qwen2-0.5B shape
// (151,936 rows of 896): HB = 2 2,516 tok/s, 1: 2,486, 3: 2,503, 4: 2,494,
// 6: 2,474; three batches of 2 in flight: 2,498.
template <int UHB>
__device__ __forceinline__ void head_dots(const uint16_t *head, float *logits, const float *xs, int H, int V, int gw,
                                          int W, int head_rows, int &key, uint32_t &idx) {
    constexpr int HB = 2;
    const int lane = lane_here(), nHB = H / 8;
    const uint32_t stride = (uint32_t)H * 2;
    const Rsrc r = rsrc(head, (size_t)V * stride);
    u32x4 hb[2][HB][UHB];
    const int nbat = (head_rows + HB - 1) / HB;
    auto issue = [&](u32x4 (&buf)[HB][UHB], int bi) {
#pragma unroll
        for (int k = 0; k < HB; ++k) {
            const int i = bi * HB + k;
            load_row(buf[k], r, (uint32_t)(gw + W * i) * stride, nHB, i < head_rows);
        }
    };
    auto consume = [&](const u32x4 (&buf)[HB][UHB], int bi) {
        const int nr = max(0, min(HB, head_rows - bi * HB));
        float y[HB];
        dot_rows<FMT_BF16>(buf, xs, nHB, y);
#pragma unroll
        for (int k = 0; k < HB; ++k)
            if (k < nr) {
                const uint32_t row = (uint32_t)(gw + W * (bi * HB + k));
                if (lane == 0) st_u32(logits + row, __float_as_uint(y[k]));
                better(key, idx, total_key(y[k]), row);
            }
    };
    issue(hb[0], 0);
    for (int bi = 0; bi < nbat; bi += 2) {
        issue(hb[1], bi + 1);
        consume(hb[0], bi);
        issue(hb[0], bi + 2);
        consume(hb[1], bi + 1);
    }
    // The last batch issued (rows past the wave's, reading nothing) is
    // retired here, so no later code inherits a wait for its registers.
    pin(hb[0]);
}


__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }
__host__ __device__ constexpr int imax(int a, int b) { return a > b ? a : b; }

// One 16-byte weight unit. A row that one block reads once per layer goes
// non-temporal (the default: it is not read again before the next step).
// The q rows and o_proj columns of a q head are read by every run of that
// head, whose blocks share one XCD: SHARED loads keep the default cache
// policy, so the first run's misses fill that XCD's L2 for the others
// (measured 2,496 vs 2,382 tok/s, the same tokens; every weight cached:
// 2,455).
template <bool SHARED = false>
__device__ __forceinline__ u32x4 ld_unit(Rsrc r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, SHARED ? 0 : 2));
}

// Wave-wide dot products of R rows held in pool slots OFF + i * N + k (unit
// k of row i in lane k % 64 of slot k / 64's register) with xs; a unit's x
// values are read once for all rows. Per row the summation order is fixed
// (unit, then element); results land in every lane. Lanes past the row
// (n_units) read a valid x at a clamped index while their weights are the
// zeros of a load that read nothing.
template <int R, int N, int OFF, int NP>
__device__ __forceinline__ void dot_pool(const u32x4 (&W)[NP], const float *xs, int n_units, float (&out)[R]) {
    static_assert(OFF + R * N <= NP, "pool slice out of range");
    using U = Unit<FMT_BF16, 16>;
    const int lane = lane_here();
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int u = min(lane + 64 * k, n_units - 1);
        float xv[U::E];
#pragma unroll
        for (int e = 0; e < U::E; ++e) xv[e] = xs[xpad(u * U::E + e)];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const u32x4 w = W[OFF + i * N + k];
            const uint32_t raw[4] = {w[0], w[1], w[2], w[3]};
            U::decode(raw, [&](int e, float v) { acc[i] = fmaf(v, xv[e], acc[i]); });
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) out[i] = wave_sum(acc[i]);
}

// ---- Matrix-core matrix-vector products.
//
// y = W x for 16 rows of W at a time with v_mfma_f32_16x16x32_bf16: the B
// operand of K-step ks is the 16 rows' BF16 elements [32 ks, 32 ks + 32),
// lane l holding 8 consecutive elements (one 16-byte weight unit, elements
// 32 ks + 8 (l / 16) ...) of row l % 16; the A operand's rows 0..2 hold x
// split into three BF16 parts (x_split), rows 3..15 zeros. Each part times
// a BF16 weight is exact in f32 and the three parts carry all 24
// significant bits of x, so the tile's output rows 0..2 add up to the f32
// dot product (lanes 0..15 hold rows 0..3 of output column l: c[0..3]).
// The VALU form needs an unpack and an FMA per element; a wave64 VALU
// instruction occupies its SIMD for 4 cycles, which made the decode's
// matrix-vector phases instruction-bound.
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

// hi = x with its low 16 bits cleared, mid = the same of x - hi, lo =
// x - hi - mid rounded to nearest even: x - hi and x - hi - mid are exact.
__device__ __forceinline__ void x_split(float x, uint16_t &hi, uint16_t &mid, uint16_t &lo) {
    hi = (uint16_t)(__float_as_uint(x) >> 16);
    const float r1 = x - bf16_f32(hi);
    mid = (uint16_t)(__float_as_uint(r1) >> 16);
    lo = f32_bf16_rne(r1 - bf16_f32(mid));
}

// The split of element i of a K-padded vector in LDS (row stride st,
// split_stride): xb[p st + i] holds part p (p < 3) and xb[3 st + i] a zero,
// the rows the A operand reads.
__device__ __forceinline__ void put_split(uint16_t *xb, int st, int i, float x) {
    uint16_t hi, mid, lo;
    x_split(x, hi, mid, lo);
    xb[i] = hi;
    xb[st + i] = mid;
    xb[2 * st + i] = lo;
    xb[3 * st + i] = 0;
}

// This lane's offset (elements) into a split vector (row stride st) for
// K-step 0: row min(lane % 16, 3), elements 8 (lane / 16) ...
__device__ __forceinline__ int a_offset(int st) {
    const int l = lane_here();
    return min(l & 15, 3) * st + 8 * (l >> 4);
}
__device__ __forceinline__ u32x4 a_frag(const uint16_t *xb, int aoff, int ks) {
    return *(const u32x4 *)(xb + aoff + 32 * ks);
}
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}
// The dot product of the tile's row `lane` (lanes 0..15).
__device__ __forceinline__ float tile_dot(f32x4 c) { return (c[0] + c[1]) + c[2]; }

// One tile over N consecutive K-steps: pool slots OFF + k against the
// split vector at xa + 32 k (xa: this lane's A offset, a_offset, plus the
// first K-step's). All A operands are read first (their LDS latency once),
// and the K-steps alternate between two accumulators (two MFMA chains).
// Call with all 64 lanes active: every lane's operands enter the product
// (inside a lane-divergent branch the reads would skip lanes).
template <int N, int OFF, int NP>
__device__ __forceinline__ float kdot(const uint16_t *xa, const u32x4 (&W)[NP]) {
    static_assert(OFF + N <= NP, "pool slice out of range");
    u32x4 af[N];
#pragma unroll
    for (int k = 0; k < N; ++k) af[k] = *(const u32x4 *)(xa + 32 * k);
    // Every read issued before the first product waits for one.
#pragma unroll
    for (int k = 0; k < N; ++k) asm volatile("" : "+v"(af[k]));
    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if (k & 1) c1 = mfma_bf16(af[k], W[OFF + k], c1);
        else c0 = mfma_bf16(af[k], W[OFF + k], c0);
    }
    return tile_dot(c0) + tile_dot(c1);
}

// The tile's 16 row values (lanes 0..15) stored two rows per 16-byte
// store: lane 2 j stores rows 2 j and 2 j + 1 at dst(2 j) (rows r < n).
template <class D>
__device__ __forceinline__ void store_tile(float y, int r0, int n, unsigned tag, D &&dst) {
    const float nb = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, y), 0xB1, 0xF, 0xF,
                                                                         true));  // quad_perm [1,0,3,2]
    const int l = lane_here(), r = r0 + l;
    if (l < 16 && (l & 1) == 0 && r < n) stf2(dst(r), y, nb, tag);
}

template <int HD>
struct ItemShm {
    // Per-wave attention partials (item_flash), the new position's last:
    // weighted V rows relative to the partial's own max, that max, and the
    // sum of the weights.
    float red[kWaves + 1][HD];
    float mw[kWaves + 1], lw[kWaves + 1];
    alignas(16) uint16_t op[4][split_stride(HD)];  // the unnormalised output, split (put_split)
    float m, l;            // max score, sum of weights
};

// Dynamic LDS layout (byte offsets): tagged-word staging, the f32 vector
// the VALU dot products read, its split for the matrix-core products (4
// rows of H padded to 32), an item's q (with its biases and rotation
// factors), its K and V rows, the embedding row, and two RMSNorm gain rows
// (BF16): g1 for the items' and KV blocks' input norm, g2 for the FFN norm
// and the final norm.
struct LdsLayout {
    int tbw;  // staging words
    int xs, xb, q, kv, emb, g1, g2, total;
};
__host__ __device__ inline LdsLayout lds_layout(int H, int hd, int kv_bytes, int ip, int ni, int nbd, int blocks) {
    LdsLayout o{};
    int tbw = imax(imax(H, round_up(ni * kOwn, kChunk) + 2 * ni), imax(nbd * kOwn, imax(2 * hd, 2 * blocks)));
    o.tbw = round_up(tbw + 2, kChunk);
    o.xs = o.tbw * 8;
    o.xb = o.xs + round_up((xpad(H) + 10) * 4, 16);
    o.q = o.xb + 4 * split_stride(round_up(H, 32)) * 2;
    o.kv = o.q + round_up(3 * hd * 4, 16);
    o.emb = o.kv + round_up(2 * ip * hd * kv_bytes, 16);
    o.g1 = o.emb + round_up(H * 2, 16);
    o.g2 = o.g1 + round_up(H * 2, 16);
    o.total = o.g2 + round_up(H * 2, 16);
    return o;
}

// Starts the copies of the cached K and V rows of positions [start, lim) of
// KV head g into LDS (row p - start of each), 1 KB pieces spread over the
// waves; completion is awaited with wait_vm. start is page-aligned.
template <int HD, class KT>
__device__ __forceinline__ void load_kv_lds(CArgs *a, uint8_t *k_lds, uint8_t *v_lds, int l, int g, long start,
                                            long lim) {
    constexpr int ROW = HD * (int)sizeof(KT);
    const int lane = lane_here(), wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    for (long t0 = start; t0 < lim; t0 += TP) {
        const int page = ldc(opaque(a)->page_table, t0 / TP);
        const int bytes = (int)(min((long)TP, lim - t0)) * ROW;
        const size_t off = (((size_t)page * opaque(a)->kv_heads + g) * TP) * ROW;
        const uint8_t *ks = (const uint8_t *)layer_of(a, l)->kc + off, *vs = (const uint8_t *)layer_of(a, l)->vc + off;
        uint8_t *kd = k_lds + (t0 - start) * ROW, *vd = v_lds + (t0 - start) * ROW;
        for (int c = wave * 1024; c < bytes; c += kWaves * 1024) {
            const int byte = c + lane * 16;
            if (byte < bytes) {
                dma16_nc(ks + byte, kd + c);
                dma16_nc(vs + byte, vd + c);
            }
        }
    }
}

// ---- An item's attention, flash style: no wave waits for another until
// the partials merge.
//
// item_flash: wave w takes the cached positions [w cw, min(w cw + cw, nc)),
// cw = ceil(nc / 8) <= 32: scores with eight lanes per position (lane i
// reads bytes 128 r + 16 i of the K row, so the eight lanes of a position
// cover 128 contiguous bytes per read, conflict-free), its own max m_w,
// weights exp(s - m_w) and their sum l_w, then the weighted V rows (lane:
// HD / 64 dimensions; a position's weight read from the lane that scored
// it) into sh.red[w], sh.mw[w], sh.lw[w]. A wave without positions leaves
// m_w = -inf, l_w = 0 and zeros.
template <int HD, class KT>
__device__ __forceinline__ void item_flash(const float *qs, const uint8_t *k_lds, const uint8_t *v_lds, int nc,
                                           ItemShm<HD> &sh) {
    constexpr int ROW = HD * (int)sizeof(KT);
    constexpr int NR = ROW / 128;              // 16-byte reads per lane and row
    constexpr int EPR = 16 / (int)sizeof(KT);  // elements per read
    constexpr int DV = HD / 64;                // V dimensions per lane
    constexpr int NPASS = kIpMax / kWaves / 8;  // passes of 8 positions, at most
    static_assert(NR >= 1 && NPASS <= 4, "row and run shape");
    const int lane = lane_here(), li = lane & 7, pj = lane >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int cw = (nc + kWaves - 1) / kWaves;
    const int p0 = wave * cw, cnt = max(0, min(cw, nc - p0));
    const float scale = 1.0f / sqrtf((float)HD);
    // This lane's elements of q: (128 r + 16 li) / sizeof(KT) + e.
    float qv[NR][EPR];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int e = 0; e < EPR; ++e) qv[r][e] = qs[(128 * r + 16 * li) / (int)sizeof(KT) + e];
    float sc[NPASS];
    float mx = -INFINITY;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
        sc[ps] = -INFINITY;
        if (8 * ps < cnt) {
            const int j = 8 * ps + pj;
            const uint8_t *krow = k_lds + (size_t)(p0 + min(j, cnt - 1)) * ROW + 16 * li;
            float dot = 0.f;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const u32x4 w = *(const u32x4 *)(krow + 128 * r);
                if constexpr (sizeof(KT) == 2) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dot = fmaf(bf16_lo(w[e]), qv[r][2 * e], dot);
                        dot = fmaf(bf16_hi(w[e]), qv[r][2 * e + 1], dot);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) dot = fmaf(__uint_as_float(w[e]), qv[r][e], dot);
                }
            }
            dot = group_sum<8>(dot);
            if (j < cnt) sc[ps] = dot * scale;
            mx = fmaxf(mx, sc[ps]);
        }
    }
    mx = wave_max(mx);
    float ew[NPASS], ls = 0.f;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
        ew[ps] = sc[ps] == -INFINITY ? 0.f : expf(sc[ps] - mx);
        if (li == 0) ls += ew[ps];
    }
    ls = wave_sum(ls);
    float acc[DV];
#pragma unroll
    for (int e = 0; e < DV; ++e) acc[e] = 0.f;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
        if (8 * ps < cnt) {
            float vf[8][DV];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const KT *vrow = (const KT *)(v_lds + (size_t)(p0 + min(8 * ps + jj, cnt - 1)) * ROW) + lane * DV;
                if constexpr (sizeof(KT) == 2) {
                    if constexpr (DV == 1) {
                        vf[jj][0] = bf16_f32(*vrow);
                    } else {
                        const uint32_t w2 = *(const uint32_t *)vrow;
                        vf[jj][0] = bf16_lo(w2);
                        vf[jj][1] = bf16_hi(w2);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < DV; ++e) vf[jj][e] = vrow[e];
                }
            }
            // Positions past the run weigh zero (their lanes hold ew = 0).
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const float w = lane_read(ew[ps], 8 * jj);
#pragma unroll
                for (int e = 0; e < DV; ++e) acc[e] = fmaf(w, vf[jj][e], acc[e]);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < DV; ++e) sh.red[wave][lane * DV + e] = acc[e];
    if (lane == 0) {
        sh.mw[wave] = mx;
        sh.lw[wave] = ls;
    }
}

// The new position's partial (sh.red/mw/lw[8]) from its K and V rows as
// stored in the cache (tagged words kv: K then V, HD each): wave 0 polls K
// and scores it against q, wave 1 polls V. Bounded like every poll.
template <int HD>
__device__ __forceinline__ void item_new_row(const float *qs, const uint64_t *kv, unsigned tag, int *abort_flag,
                                             ItemShm<HD> &sh) {
    static_assert(HD <= 2 * 64, "a row of the new position in one chunk");
    const int lane = lane_here(), wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6), d = 2 * lane;
    if (wave == 0) {
        const u32x4 r = poll_chunk(kv, 0, HD, tag, abort_flag);
        float dot = 0.f;
        if (d < HD) dot = fmaf(__uint_as_float(r[2]), qs[d + 1], __uint_as_float(r[0]) * qs[d]);
        dot = wave_sum(dot);
        if (lane == 0) {
            sh.mw[kWaves] = dot * (1.0f / sqrtf((float)HD));
            sh.lw[kWaves] = 1.f;
        }
    } else if (wave == 1) {
        const u32x4 r = poll_chunk(kv + HD, 0, HD, tag, abort_flag);
        if (d < HD) {
            sh.red[kWaves][d] = __uint_as_float(r[0]);
            sh.red[kWaves][d + 1] = __uint_as_float(r[2]);
        }
    }
}

// Threads d < HD, after a barrier: the partials (the waves', then the new
// position's when there is one) rescaled to their common max and added in
// that order: the unnormalised output split into sh.op, sh.m, sh.l. Lane w
// of each wave computes partial w's factor exp(m_w - M) (one exponential
// per lane), the others read it from there.
template <int HD>
__device__ __forceinline__ void item_merge(bool has_new, ItemShm<HD> &sh) {
    constexpr int NP = kWaves + 1;
    const int tid = tid_here(), lane = tid & 63;
    if (tid < HD) {
        const int np = kWaves + (has_new ? 1 : 0);
        const int li = min(lane, NP - 1);
        const float mw = lane < np ? sh.mw[li] : -INFINITY;
        const float M = wave_max(mw);
        const float f = mw == -INFINITY ? 0.f : expf(mw - M);
        const float l = wave_sum(lane < np ? f * sh.lw[li] : 0.f);
        // (The new position's slot holds nothing to read when there is none.)
        float rv[NP];
#pragma unroll
        for (int w = 0; w < NP; ++w) rv[w] = w < np ? sh.red[w][tid] : 0.f;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < NP; ++w) o = fmaf(lane_read(f, w), rv[w], o);
        put_split(&sh.op[0][0], split_stride(HD), tid, o);
        if (tid == 0) {
            sh.m = M;
            sh.l = l;
        }
    }
}

// UH: 16-byte units per lane of a row with H columns (the KV blocks' and
// the LM head's VALU dot products); KS: K-steps of 32 columns of a row with
// H columns (H <= 32 KS); OTW: 16-row tiles of H rows per wave (H <= 128
// OTW); GT: 16-row tiles of an FFN block's gate (and up) rows. Shape values
// are re-read from the arguments where used (A()) and block roles
// recomputed from them, so that little stays in scalar registers across the
// step loop.
//
// Matrix-core work per wave (one 16-byte weight unit per lane and MFMA):
//   items' q and FFN gate/up: every tile (HD / 16 q tiles; GT gate and GT
//     up tiles) over the four K-steps of the wave's own input chunk (wave w
//     polls elements [128 w, 128 w + 128)), so a wave multiplies as soon as
//     its chunk is in, with no barrier before; the chunks' sums meet in LDS;
//   items' o_proj: tiles wave, wave + 8, ... of the H rows, HD / 32 K-steps;
//   FFN down: tiles wave, wave + 8, ... of the H rows, one K-step (the
//     block's gate/up rows padded to 32).
//
// Each role runs its own step and layer loops (one branch per role), with
// the LM head and the token reduction shared: a loop carries only its
// role's weight registers, and a CU's hot code is only its role's.
template <int HD, int G, class KT, int UH, int KS, int OTW, int GT>
__global__ __launch_bounds__(kThreads) void decode_flow_kernel(FusedArgs) {
    using U = Unit<FMT_BF16, 16>;
    constexpr int ROW = HD * (int)sizeof(KT);
    constexpr int KP = 32 * KS;           // padded K of a row with H columns
    constexpr int QT = HD / 16;           // q tiles of a head
    constexpr int CK = kChunk / 32;       // K-steps of one wave's input chunk
    constexpr int OK = HD / 32;           // K-steps of an o_proj row's head columns
    constexpr int NQ = QT * CK;           // an item's q units
    constexpr int NWO = OTW * OK;         // an item's o_proj units
    constexpr int NI = NQ + NWO;          // an item's weight units
    constexpr int GT2 = 2 * GT;           // gate and up tiles of an FFN block
    constexpr int NG = GT2 * CK;          // an FFN block's gate/up units
    constexpr int ND = OTW;               // an FFN block's down units
    constexpr int NF = NG + ND;           // an FFN block's weight units
    constexpr int NK = 2 * UH;            // a KV block's weight units
    static_assert(HD % 32 == 0 && QT * 16 <= 128 && GT2 * 16 <= 128 && KS <= kWaves * CK, "tiles and chunks");
    // The only read of the kernarg-segment pointer (see opaque()).
    CArgs *const kargs = (CArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    auto A = [kargs]() { return opaque(kargs); };
    auto LY = [kargs](int l) { return layer_of(kargs, l); };
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ Shm sm;
    __shared__ ItemShm<HD> ish;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int b = blockIdx.x;
    uint64_t *tb = (uint64_t *)lds;

    // Roles: items (split s, head h) at block s * heads_padded + slot(h)
    // for s < splits (item index s * q_heads + h), KV blocks
    // [kv0, kv0 + nkv) (wave w of KV block k: rotation pair 8 k + w of the
    // K/V rows), FFN blocks [f0, f0 + nf): block f owns gate/up rows
    // [f rb, f rb + rb) (wave w rows w, w + 8, ...) and, for f < no, the
    // residual rows 8 f + w. Blocks in none of these only join the LM head.
    auto slotHead = [&]() { return (int)A()->slot_head[b % heads_padded(A()->q_heads)]; };
    auto isItem = [&]() { return b < A()->splits * heads_padded(A()->q_heads) && slotHead() >= 0; };
    auto isKV = [&]() { return b >= A()->kv0 && b < A()->kv0 + A()->nkv; };
    auto fIdx = [&]() { return b - A()->f0; };
    auto isFFN = [&]() { return b >= A()->f0; };
    auto isOwner = [&]() { return isFFN() && fIdx() < A()->no; };
    auto hasRows = [&]() { return isFFN() && fIdx() < A()->nbd; };
    auto hasHead = [&]() { return b * kWaves < A()->V; };
    auto itHead = [&]() { return slotHead(); };
    auto itSplit = [&]() { return b / heads_padded(A()->q_heads); };
    auto itIdx = [&]() { return itSplit() * A()->q_heads + itHead(); };
    auto kvPair = [&]() { return (b - A()->kv0) * kWaves + wave; };
    auto ownRow = [&]() { return fIdx() * kOwn + wave; };

    // Optional per-phase timestamps of one step (thread 0 of each block).
    auto mark = [&](int step, int ev) {
        if (A()->trace && step == A()->trace_step && tid_here() == 0)
            st_u64(A()->trace + (size_t)b * (16 * A()->L + 3) + ev, wall_clock64());
    };
    // A phase's normed input: every wave computes the scale itself (same
    // order, same value) and stages its share of xs.
    auto stage_norm = [&](const void *src, bool bf16_src, int gain_off) {
        const uint16_t *g = (const uint16_t *)(lds + gain_off);
        float *xs = (float *)(lds + A()->lds_xs);
        const int H = A()->H;
        if (bf16_src) block_stage<true>(xs, src, H, g, wave_norm_scale<true>(src, H, A()->eps));
        else block_stage<false>(xs, src, H, g, wave_norm_scale<false>(src, H, A()->eps));
    };
    // A normed input for the matrix-core products, in two halves: before
    // the barrier, wave w takes elements [128 w, 128 w + 128) of the input
    // (lane l: 128 w + 2 l and + 1, values v0 and v1, gains gw as two BF16
    // halves), writes the split of x * g into xb (two elements per LDS
    // store; zeros past H up to KP) and its sum of squares into sm.ss[w];
    // after it, norm_scale() folds the eight sums in wave order into the
    // RMSNorm scale (ops.rs:646-652), which multiplies the dot products of
    // x * g (the same value as the dot product of the normed x up to one
    // rounding). No wave waits for another between its input and its
    // share of xb, and the block passes one barrier on the way to the
    // products.
    auto stage_gx = [&](float v0, float v1, uint32_t gw) {
        const int H = A()->H, lane = lane_here(), base = wave * kChunk, i0 = base + 2 * lane;
        float ss = 0.f;
        if (base < H) {
            ss = wave_sum(fmaf(v1, v1, v0 * v0));
            // Elements [H, KP) are zeros: they lie in the chunk that holds H - 1.
            if (i0 < KP) {
                uint16_t a[3], c[3];
                x_split(v0 * bf16_lo(gw), a[0], a[1], a[2]);
                x_split(v1 * bf16_hi(gw), c[0], c[1], c[2]);
                uint32_t *xb = (uint32_t *)(lds + A()->lds_xb);
                constexpr int st = split_stride(KP) / 2;  // row stride in 32-bit words
#pragma unroll
                for (int p = 0; p < 3; ++p) xb[p * st + i0 / 2] = (uint32_t)a[p] | ((uint32_t)c[p] << 16);
                xb[3 * st + i0 / 2] = 0u;
            }
        }
        if (lane == 0) sm.ss[wave] = ss;
    };
    auto norm_scale = [&]() {
        float tot = sm.ss[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) tot += sm.ss[w];
        return 1.0f / sqrtf(tot / (float)A()->H + A()->eps);
    };
    // This wave's products of NT tiles (pool slots OFF + t CK + k) over the
    // K-steps of its own input chunk (staged in xb by stage_gx, read back by
    // the same wave: no barrier), tile t's 16 outputs into sm.red[wave][16 t
    // + lane]. Every lane takes part (the products read all 64 lanes).
    auto chunk_products = [&](auto nt_c, auto off_c, const u32x4 *W) {
        constexpr int NT = decltype(nt_c)::value, OFF = decltype(off_c)::value;
        const uint16_t *xa = (const uint16_t *)(lds + A()->lds_xb) + a_offset(split_stride(KP)) + 32 * CK * wave;
        u32x4 af[CK];
#pragma unroll
        for (int k = 0; k < CK; ++k) {
            af[k] = u32x4{0u, 0u, 0u, 0u};
            if (CK * wave + k < KS) af[k] = *(const u32x4 *)(xa + 32 * k);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f32x4 c = {0.f, 0.f, 0.f, 0.f};
            // K-steps past KS hold zeros on both sides (no read, no load).
#pragma unroll
            for (int k = 0; k < CK; ++k) c = mfma_bf16(af[k], W[OFF + t * CK + k], c);
            if (lane_here() < 16) sm.red[wave][16 * t + lane_here()] = tile_dot(c);
        }
    };
    // Input chunks of H: the waves whose sums sm.red holds.
    auto n_chunks = [&]() { return (A()->H + kChunk - 1) / kChunk; };
    // This wave's input values from the tagged words src (chunk `wave`,
    // polled into registers; zeros past H).
    auto poll_x = [&](const uint64_t *src, unsigned tag, float &v0, float &v1) {
        const int H = A()->H, base = wave * kChunk, i0 = base + 2 * lane_here();
        v0 = v1 = 0.f;
        if (base < H) {
            const u32x4 r = poll_chunk(src, base, H, tag, A()->abort_flag);
            v0 = i0 < H ? __uint_as_float(r[0]) : 0.f;
            v1 = i0 + 1 < H ? __uint_as_float(r[2]) : 0.f;
        }
    };
    // The gains of this lane's two input elements (a BF16 pair), loaded with
    // the layer's weights.
    auto load_gains = [&](const uint16_t *g, bool act) {
        const int H = A()->H, i0 = wave * kChunk + 2 * lane_here();
        const uint32_t off = act && i0 < H ? (uint32_t)i0 * 2u : kNoRead;
        return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsrc(g, (size_t)H * 2), off, 0, 2);
    };
    auto tag_base = [&](int s) { return A()->tag0 + (unsigned)(s * fused_phases_per_step(A()->L)); };

    // The LM head of step s (BF16, final norm fused) and this block's argmax
    // partial (key, index), by step parity.
    auto lm_head = [&](int s) {
        const int L = A()->L;
        const unsigned tH = tag_base(s) + 5 * L;
        int key = INT_MIN;
        uint32_t idx = 0;
        if (hasHead()) {
            if (wave == kDmaWave) dma_bytes(lds + A()->lds_g2, A()->final_norm, A()->H * 2);
            gather(tb, A()->hid1, A()->H, tH - 1, A()->abort_flag);
            wait_vm();
            bar();
            stage_norm(tb, false, A()->lds_g2);
            bar();
            mark(s, 16 * L);
            const int Wn = (int)gridDim.x * kWaves, gw0 = b * kWaves + wave, V = A()->V;
            const int head_rows = gw0 < V ? (V - 1 - gw0) / Wn + 1 : 0;
            head_dots<UH>(A()->head, A()->logits, (const float *)(lds + A()->lds_xs), A()->H, V, gw0, Wn, head_rows,
                           key, idx);
        }
        block_best(key, idx, sm);
        mark(s, 16 * L + 1);
        uint64_t *am = A()->am + (size_t)(s & 1) * gridDim.x * 2;
        if (hasHead() && tid_here() == 0) {
            stt(am + 2 * b, (uint32_t)key, tH);
            stt(am + 2 * b + 1, idx, tH);
        }
    };
    // Blocks that use the token (embedding row, residual) reduce step s's
    // argmax partials of every head block into the token at position
    // pos + 1 (block 0 records it). A partial that never arrived (the poll
    // gave up) still holds a valid row index; the token then keeps its last
    // value.
    auto reduce_token = [&](int s, long pos, int token) {
        const int head_blocks = A()->head_blocks;
        uint64_t *am = A()->am + (size_t)(s & 1) * gridDim.x * 2;
        gather(tb, am, 2 * head_blocks, tag_base(s) + 5 * A()->L, A()->abort_flag);
        bar();
        if (wave == 0) {
            int key = INT_MIN;
            uint32_t idx = 0;
            for (int i = lane_here(); i < head_blocks; i += 64)
                better(key, idx, (int)(uint32_t)tb[2 * i], (uint32_t)tb[2 * i + 1]);
            wave_best(key, idx);
            if (lane_here() == 0) sm.token = idx < (uint32_t)A()->V ? (int)idx : token;
        }
        bar();
        token = __builtin_amdgcn_readfirstlane(sm.token);
        if (b == 0 && tid_here() == 0) {
            if (pos + 1 < A()->hist_cap) st_u32(A()->hist + pos + 1, (uint32_t)token);
            st_u32(A()->step, (uint32_t)token);
            st_u32(A()->step + 1, (uint32_t)(pos + 1));
        }
        mark(s, 16 * A()->L + 2);
        return token;
    };

    int token = __builtin_amdgcn_readfirstlane(__hip_atomic_load(A()->step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const long pos0 =
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(A()->step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));

    if (isItem()) {
        // ---- Items: one q head over one run of positions. Per layer: the
        // input (fused RMSNorm), the head's 64 q rows (bias, RoPE), scores
        // of the run's cached K rows, the new position's K/V row from the
        // KV blocks (the run that holds it), softmax, weighted V rows, and
        // the head's o_proj columns applied to the unnormalised output.
        u32x4 W[NI];
        uint32_t gw1 = 0;  // input-norm gains of this lane's two elements
        // Refill for layer l at position pos: q units (k < NQ: tile k / CK,
        // row 16 (k / CK) + lane % 16 of the head, K-step ks = CK wave +
        // k % CK of the wave's input chunk, unit 4 ks + lane / 16), o_proj units
        // (k = NQ + m OK + j: tile wave + 8 m of the H rows, row 16 t +
        // lane % 16, K-step j of the head's columns, elements
        // h HD + 32 j + 8 (lane / 16) ...), the input-norm gains and the
        // run's cached K/V rows (when `act`).
        auto refill = [&](int l, bool act, long pos) {
            const int H = A()->H, nH = H / U::E, lane = lane_here(), i16 = lane & 15, g4 = lane >> 4;
            const uint32_t qs = (uint32_t)A()->qkv_stride, os = (uint32_t)A()->o_stride;
            const int qrows = (A()->q_heads + 2 * A()->kv_heads) * HD;
            const Rsrc rq = rsrc(LY(l)->qkv, (size_t)qrows * qs), ro = rsrc(LY(l)->o, (size_t)H * os);
            const int h = itHead();
            gw1 = load_gains(LY(l)->ln1, act);
#pragma unroll
            for (int k = 0; k < NI; ++k) {
                uint32_t off = kNoRead;
                if (k < NQ) {
                    const int ks = CK * wave + k % CK, unit = 4 * ks + g4, row = h * HD + (k / CK) * 16 + i16;
                    if (act && ks < KS && unit < nH) off = (uint32_t)row * qs + (uint32_t)unit * 16u;
                    W[k] = ld_unit<true>(rq, off);
                } else {
                    const int m = (k - NQ) / OK, j = (k - NQ) % OK, r = (wave + kWaves * m) * 16 + i16;
                    if (act && r < H) off = (uint32_t)r * os + (uint32_t)(h * HD + 32 * j + 8 * g4) * 2u;
                    W[k] = ld_unit<true>(ro, off);
                }
            }
            if (act) {
                const int ip = A()->ip;
                const long start = (long)itSplit() * ip, lim = min(start + ip, pos);
                uint8_t *k_lds = lds + A()->lds_kv;
                load_kv_lds<HD, KT>(kargs, k_lds, k_lds + ip * ROW, l, itHead() / G, start, lim);
            }
        };
        long pos = pos0;
        // Layer 0's rows of a step after the first are loaded at the end of
        // the step before (after its last layer's partials, while the block
        // waits for the LM head's input), so that the token's poll at the
        // step's start has no refill in front of it (a wave's loads complete
        // in order).
        bool primed = false;
        for (int s = 0;; ++s) {
            const bool run = s < A()->steps;
            const int L = A()->L, ip = A()->ip;
            const long ctx = pos + 1;
            const int S = (int)((ctx + ip - 1) / ip);
            // This block's run: q head ih, positions [kv_start, kv_end); rows
            // below nc are cached, the new one comes tagged.
            const bool active = run && itSplit() < S;
            const int ih = itHead();
            const long kv_start = (long)itSplit() * ip, kv_end = min(kv_start + ip, ctx);
            const int nc = active ? (int)(min(kv_end, pos) - kv_start) : 0;
            const bool has_new = active && kv_end == ctx;
            const unsigned tb0 = tag_base(s);
            if (!primed) refill(0, active, pos);
            if (s > 0) token = reduce_token(s - 1, pos - 1, token);
            if (!run) break;
            if (wave == kDmaWave) dma_bytes(lds + A()->lds_emb, A()->embed + (size_t)token * A()->H, A()->H * 2);
            for (int l = 0; l < L; ++l) {
                const unsigned tK = tb0 + 5 * l, tP = tK + 1;
                mark(s, 16 * l);
                if (active) {
                    float *qs = (float *)(lds + A()->lds_q);  // q[hd], bias[hd], cos[hd / 2], sin[hd / 2]
                    uint8_t *k_lds = lds + A()->lds_kv, *v_lds = k_lds + ip * ROW;
                    const int H = A()->H, rot = A()->rotary, half = rot / 2;
                    // q's biases (rows of head ih, pair-permuted like the
                    // rows) and rotation factors, loaded before the poll.
                    const float *qbias = LY(l)->qkv_bias;
                    {
                        const int tid = tid_here();
                        if (tid < HD) {
                            qs[HD + tid] = qbias ? qbias[ih * HD + tid] : 0.f;
                        } else if (tid < HD + half) {
                            const int i = tid - HD;
                            qs[2 * HD + i] = A()->rope_cos[pos * half + i];
                            qs[2 * HD + HD / 2 + i] = A()->rope_sin[pos * half + i];
                        }
                    }
                    // (wait_vm: the embedding row and the K/V rows)
                    float x0, x1;
                    if (l > 0) {
                        poll_x(A()->hid1, tK - 1, x0, x1);
                    } else {
                        wait_vm();
                        bar();
                        const int i0 = wave * kChunk + 2 * lane_here();
                        const uint16_t *e = (const uint16_t *)(lds + A()->lds_emb);
                        x0 = i0 < H ? bf16_f32(e[i0]) : 0.f;
                        x1 = i0 + 1 < H ? bf16_f32(e[i0 + 1]) : 0.f;
                    }
                    stage_gx(x0, x1, gw1);
                    mark(s, 16 * l + 1);
                    {
                        // The head's q rows on the matrix cores over this
                        // wave's chunk; the chunks' sums added in wave order.
                        chunk_products(std::integral_constant<int, QT>{}, std::integral_constant<int, 0>{}, W);
                        wait_vm();
                        bar();
                        // Thread j < HD / 2 finishes rotation pair j (rows
                        // 2 j and 2 j + 1: norm scale, bias, RoPE).
                        const int tid = tid_here();
                        if (tid < HD / 2) {
                            const int d0 = 2 * tid, nch = n_chunks();
                            float v0 = sm.red[0][d0], v1 = sm.red[0][d0 + 1];
                            for (int w = 1; w < nch; ++w) {
                                v0 += sm.red[w][d0];
                                v1 += sm.red[w][d0 + 1];
                            }
                            const float inv = norm_scale();
                            v0 = inv * v0;
                            v1 = inv * v1;
                            if (qbias) {
                                v0 = v0 + qs[HD + d0];
                                v1 = v1 + qs[HD + d0 + 1];
                            }
                            if (d0 < rot) {
                                const int i = d0 / 2;
                                const float c = qs[2 * HD + i], sn = qs[2 * HD + HD / 2 + i];
                                qs[i] = v0 * c - v1 * sn;
                                qs[half + i] = v1 * c + v0 * sn;
                            } else {
                                qs[d0] = v0;
                                qs[d0 + 1] = v1;
                            }
                        }
                    }
                    bar();
                    mark(s, 16 * l + 2);
                    // Attention: the waves' partials over the cached rows,
                    // the new position's (its K and V rows as stored in the
                    // cache, from the KV blocks), then one merge.
                    item_flash<HD, KT>(qs, k_lds, v_lds, nc, ish);
                    mark(s, 16 * l + 3);
                    if (has_new) item_new_row<HD>(qs, A()->kvw + (size_t)(ih / G) * 2 * HD, tK, A()->abort_flag, ish);
                    mark(s, 16 * l + 4);
                    bar();
                    item_merge<HD>(has_new, ish);
                    bar();
                    mark(s, 16 * l + 5);
                    // o_proj columns of head ih times the unnormalised output
                    // on the matrix cores: tiles wave + 8 m of the H rows
                    // over the head's OK K-steps, each row stored as owner
                    // r / 8's partial of item b (two rows per store); the
                    // run's max and sum once.
                    {
                        const int aoff = a_offset(split_stride(HD));
                        u32x4 oa[OK];
#pragma unroll
                        for (int j = 0; j < OK; ++j) oa[j] = a_frag(&ish.op[0][0], aoff, j);
                        const int ni = A()->ni, it = __builtin_amdgcn_readfirstlane(itIdx());
                        uint64_t *part = A()->part + (size_t)it * kOwn;
                        f32x4 acc[OTW];
#pragma unroll
                        for (int m = 0; m < OTW; ++m) {
                            acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int j = 0; j < OK; ++j) acc[m] = mfma_bf16(oa[j], W[NQ + m * OK + j], acc[m]);
                        }
#pragma unroll
                        for (int m = 0; m < OTW; ++m)
                            store_tile(tile_dot(acc[m]), (wave + kWaves * m) * 16, H, tP, [&](int r) {
                                return part + (size_t)(r / kOwn) * ni * kOwn + r % kOwn;
                            });
                        if (tid_here() == 0) stf2(A()->ml + 2 * it, ish.m, ish.l, tP);
                    }
                    bar();
                    mark(s, 16 * l + 6);
                }
                if (l + 1 < L) {
                    refill(l + 1, active, pos);
                } else if (s + 1 < A()->steps) {
                    // The next step's layer 0 at position pos + 1 (context
                    // pos + 2): its cached rows, up to position pos, are
                    // all written by now.
                    refill(0, itSplit() < (int)((pos + 1 + ip) / ip), pos + 1);
                }
            }
            primed = s + 1 < A()->steps;
            lm_head(s);
            ++pos;
        }
    } else if (isKV()) {
        // ---- KV blocks: the new position's K and V rows (fused RMSNorm,
        // bias, RoPE), appended to the pages and handed to the items.
        u32x4 W[NK];
        auto refill = [&](int l, bool act) {
            const int H = A()->H, nH = H / U::E, lane = lane_here();
            const int qd = A()->q_heads * HD, kvd = A()->kv_heads * HD;
            const uint32_t qs = (uint32_t)A()->qkv_stride;
            const Rsrc rq = rsrc(LY(l)->qkv, (size_t)(qd + 2 * kvd) * qs);
            const int p = kvPair();
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const int unit = lane + 64 * (k % UH);
                const bool v = act && p < kvd && unit < nH;
                W[k] = ld_unit(rq, v ? (uint32_t)(qd + 2 * p + k / UH) * qs + (uint32_t)unit * 16u : kNoRead);
            }
            if (act && wave == kDmaWave) dma_bytes(lds + A()->lds_g1, LY(l)->ln1, H * 2);
        };
        long pos = pos0;
        for (int s = 0;; ++s) {
            const bool run = s < A()->steps;
            const int L = A()->L;
            const unsigned tb0 = tag_base(s);
            refill(0, run);
            if (s > 0) token = reduce_token(s - 1, pos - 1, token);
            if (!run) break;
            if (wave == kDmaWave) dma_bytes(lds + A()->lds_emb, A()->embed + (size_t)token * A()->H, A()->H * 2);
            for (int l = 0; l < L; ++l) {
                const unsigned tK = tb0 + 5 * l;
                mark(s, 16 * l);
                const int H = A()->H, nH = H / U::E, rot = A()->rotary, half = rot / 2;
                const bool myKV = kvPair() < A()->kv_heads * HD;
                // Everything the epilogue reads besides the dot (biases,
                // rotation factors, page, destinations) is loaded before the
                // input poll.
                bool k_bias = false, k_rope = false;
                float k_b0 = 0.f, k_b1 = 0.f, k_c = 0.f, k_sn = 0.f;
                int k_i0 = 0, k_i1 = 0, k_c0 = 0, k_c1 = 0;  // K/V word, cache element (bit 30: V)
                KT *cache = nullptr;
                if (myKV) {
                    const int qd = A()->q_heads * HD, kvd = A()->kv_heads * HD, kvh = A()->kv_heads;
                    const int r0 = qd + 2 * kvPair();
                    if (const float *bias = LY(l)->qkv_bias) {
                        k_bias = true;
                        k_b0 = ldc(bias, r0);
                        k_b1 = ldc(bias, r0 + 1);
                    }
                    const int page = ldc(A()->page_table, pos / TP), slot = (int)(pos % TP);
                    if (r0 < qd + kvd) {
                        const int base = r0 - qd, hh = base / HD, d0 = base % HD;
                        int o0 = d0, o1 = d0 + 1;
                        if (d0 < rot) {
                            const int i = d0 / 2;
                            k_rope = true;
                            k_c = ldc(A()->rope_cos, pos * half + i);
                            k_sn = ldc(A()->rope_sin, pos * half + i);
                            o0 = i;
                            o1 = half + i;
                        }
                        k_i0 = hh * 2 * HD + o0;
                        k_i1 = hh * 2 * HD + o1;
                        const int e0 = ((page * kvh + hh) * TP + slot) * HD;
                        k_c0 = e0 + o0;
                        k_c1 = e0 + o1;
                    } else {
                        const int base = r0 - qd - kvd, hh = base / HD, d0 = base % HD;
                        k_i0 = hh * 2 * HD + HD + d0;
                        k_i1 = k_i0 + 1;
                        const int e0 = ((page * kvh + hh) * TP + slot) * HD;
                        k_c0 = (e0 + d0) | (1 << 30);
                        k_c1 = (e0 + d0 + 1) | (1 << 30);
                    }
                    cache = (KT *)((k_c0 >> 30) ? LY(l)->vc : LY(l)->kc);
                    asm volatile("" : "+v"(k_b0), "+v"(k_b1), "+v"(k_c), "+v"(k_sn));
                }
                if (l > 0) gather(tb, A()->hid1, H, tK - 1, A()->abort_flag);
                wait_vm();  // the embedding row and the gains
                bar();
                if (l == 0) stage_norm(lds + A()->lds_emb, true, A()->lds_g1);
                else stage_norm(tb, false, A()->lds_g1);
                bar();
                mark(s, 16 * l + 1);
                {
                    float y[2];
                    dot_pool<2, UH, 0>(W, (const float *)(lds + A()->lds_xs), nH, y);
                    float v0 = y[0], v1 = y[1];
                    if (k_bias) {
                        v0 = v0 + k_b0;
                        v1 = v1 + k_b1;
                    }
                    if (k_rope) {
                        const float x1 = v0 * k_c - v1 * k_sn, x2 = v1 * k_c + v0 * k_sn;
                        v0 = x1;
                        v1 = x2;
                    }
                    if (myKV && lane_here() == 0) {
                        st_kv(cache + (k_c0 & ((1 << 30) - 1)), v0);
                        st_kv(cache + (k_c1 & ((1 << 30) - 1)), v1);
                        uint64_t *kvw = A()->kvw;
                        stf(kvw + k_i0, kv_round<KT>(v0), tK);
                        stf(kvw + k_i1, kv_round<KT>(v1), tK);
                    }
                }
                mark(s, 16 * l + 6);
                if (l + 1 < L) refill(l + 1, true);
            }
            lm_head(s);
            ++pos;
        }
    } else {
        // ---- FFN blocks (and blocks with no role, which only join the LM
        // head). Per layer: owners merge every head's runs and add the
        // residual; blocks with gate/up rows run gate/up (fused RMSNorm),
        // SwiGLU and their down columns; owners sum the down partials and
        // add the residual.
        u32x4 W[NF];
        uint32_t gw2 = 0;  // FFN-norm gains of this lane's two elements
        // Refill for layer l: gate/up units (k < NG: tile T = k / CK, gate
        // tiles first, then up; K-step ks = CK wave + k % CK of the wave's
        // input chunk; row f rb + 16 (T % GT) + lane % 16, unit 4 ks +
        // lane / 16), down units
        // (k = NG + m: tile wave + 8 m of the H rows, row 16 t + lane % 16
        // of the block's down_cols, unit lane / 16) and the gains of the FFN
        // norm.
        auto refill = [&](int l, bool act) {
            const int H = A()->H, nH = H / U::E, lane = lane_here(), i16 = lane & 15, g4 = lane >> 4;
            const uint32_t gs = (uint32_t)A()->gu_stride;
            const int rb = A()->rb, rp = A()->rp, f = fIdx(), I = A()->I;
            const Rsrc rg = rsrc(LY(l)->gate, (size_t)I * gs), ru = rsrc(LY(l)->up, (size_t)I * gs);
            const Rsrc rd = rsrc(LY(l)->down_cols, (size_t)A()->nf * H * rp * 2);
            gw2 = load_gains(LY(l)->ln2, act);
#pragma unroll
            for (int k = 0; k < NF; ++k) {
                uint32_t off = kNoRead;
                if (k < NG) {
                    const int T = k / CK, jj = (T % GT) * 16 + i16, row = f * rb + jj;
                    const int ks = CK * wave + k % CK, unit = 4 * ks + g4;
                    if (act && jj < rb && row < I && ks < KS && unit < nH) off = (uint32_t)row * gs + (uint32_t)unit * 16u;
                    W[k] = ld_unit(T < GT ? rg : ru, off);
                } else {
                    const int r = (wave + kWaves * (k - NG)) * 16 + i16;
                    if (act && r < H && g4 * 8 < rp) off = ((uint32_t)(f * H + r) * (uint32_t)rp) * 2u + (uint32_t)g4 * 16u;
                    W[k] = ld_unit(rd, off);
                }
            }
        };
        long pos = pos0;
        float h_own = 0.f, emb_r = 0.f;
        for (int s = 0;; ++s) {
            const bool run = s < A()->steps;
            const int L = A()->L, ip = A()->ip;
            const int S = (int)((pos + ip) / ip);  // ceil((pos + 1) / ip)
            const unsigned tb0 = tag_base(s);
            if (s > 0 && isOwner()) token = reduce_token(s - 1, pos - 1, token);
            if (!run) break;
            if (isOwner() && ownRow() < A()->H) emb_r = ldc_bf16(A()->embed, (long)token * A()->H + ownRow());
            for (int l = 0; l < L; ++l) {
                const unsigned tK = tb0 + 5 * l, tP = tK + 1, tC = tK + 2, tD = tK + 3, tE = tK + 4;
                const int H = A()->H;
                mark(s, 16 * l);
                refill(l, hasRows());
                mark(s, 16 * l + 7);

                // ---- Owners: every head's runs merged in split order (lane
                // h: weights exp(m_s - M), sum L = sum_s w_s l_s), + residual.
                if (isOwner()) {
                    const int Q = A()->q_heads, ni = A()->ni, r = ownRow();
                    // The o_proj bias of the row, loaded before the poll.
                    const float *ob = LY(l)->o_bias;
                    const bool has_ob = ob != nullptr && r < H;
                    float obv = has_ob ? ldc(ob, r) : 0.f;
                    asm volatile("" : "+v"(obv));
                    const int na = S * Q * kOwn;
                    gather(tb, Ranges{A()->part + (size_t)fIdx() * ni * kOwn, A()->ml, na, 2 * S * Q}, tP,
                           A()->abort_flag);
                    bar();
                    mark(s, 16 * l + 8);
                    float contrib = 0.f;
                    const int ln = lane_here();
                    {
                        // Lane (k, h) = (ln / HP, ln % HP), HP the q heads
                        // rounded up to 16, 32 or 64, takes head h's runs
                        // k, k + 64 / HP, ...: their maxima, sums and this
                        // row's partials (16-byte reads of the max and sum
                        // pairs); the lanes of one head then agree on its max
                        // M_h, weigh their runs by exp(m_s - M_h) and add up
                        // across lanes (xor shuffles), and lanes k = 0 hold
                        // the head's output A_h / L_h.
                        const int HP = Q <= 16 ? 16 : (Q <= 32 ? 32 : 64), SP = 64 / HP;
                        const int h = ln & (HP - 1), k = ln / HP;
                        const uint64_t *ml = tb + round_up(na, kChunk);
                        float mv[kMaxSplits], lv[kMaxSplits], pv[kMaxSplits], mloc = -INFINITY;
#pragma unroll
                        for (int c = 0; c < kMaxSplits; ++c) {
                            mv[c] = -INFINITY;
                            lv[c] = pv[c] = 0.f;
                            if (c * SP < S) {
                                const int sp = c * SP + k;
                                const int it = min(sp, S - 1) * Q + min(h, Q - 1);
                                const u32x4 pair = *(const u32x4 *)(ml + 2 * it);
                                const float pp = val_of(tb[it * kOwn + wave]);
                                if (h < Q && sp < S) {
                                    mv[c] = __uint_as_float(pair[0]);
                                    lv[c] = __uint_as_float(pair[2]);
                                    pv[c] = pp;
                                }
                                mloc = fmaxf(mloc, mv[c]);
                            }
                        }
                        for (int off = HP; off < 64; off <<= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off, 64));
                        float A = 0.f, Lh = 0.f;
#pragma unroll
                        for (int c = 0; c < kMaxSplits; ++c) {
                            if (c * SP < S) {
                                const float f = mv[c] == -INFINITY ? 0.f : expf(mv[c] - mloc);
                                A = fmaf(f, pv[c], A);
                                Lh = fmaf(f, lv[c], Lh);
                            }
                        }
                        for (int off = HP; off < 64; off <<= 1) {
                            A += __shfl_xor(A, off, 64);
                            Lh += __shfl_xor(Lh, off, 64);
                        }
                        if (k == 0 && h < Q) contrib = A * (1.0f / Lh);
                    }
                    const float o = wave_sum(contrib);
                    if (r < H) {
                        float v = o;
                        if (has_ob) v = v + obv;
                        h_own = (l == 0 ? emb_r : h_own) + v;
                        if (lane_here() == 0) sm.out[wave] = h_own;
                    }
                    bar();
                    const int cnt = min(kOwn, H - fIdx() * kOwn);
                    // Stored by the wave that polls no chunk of the gather
                    // that follows: a poll's wait also waits for the
                    // acknowledgement of its own wave's stores.
                    if (wave == kDmaWave && lane_here() < cnt)
                        stf(A()->hid0 + fIdx() * kOwn + lane_here(), sm.out[lane_here()], tC);
                    mark(s, 16 * l + 9);
                }

                // ---- Gate/up (fused RMSNorm), SwiGLU, down partials of every
                // hidden row.
                if (hasRows()) {
                    float x0, x1;
                    poll_x(A()->hid0, tC, x0, x1);
                    stage_gx(x0, x1, gw2);
                    mark(s, 16 * l + 10);
                    const int rb = A()->rb, f = fIdx(), I = A()->I;
                    {
                        // Gate and up rows on the matrix cores over this
                        // wave's chunk; the chunks' sums added in wave order.
                        chunk_products(std::integral_constant<int, GT2>{}, std::integral_constant<int, 0>{}, W);
                        wait_vm();
                        bar();
                        // Thread j < 32: SwiGLU of the block's row j (zero
                        // past its rows), split for the down product.
                        const int tid = tid_here();
                        if (tid < 32) {
                            float v = 0.f;
                            if (tid < rb && f * rb + tid < I) {
                                const int nch = n_chunks();
                                float gv = sm.red[0][tid], uv = sm.red[0][16 * GT + tid];
                                for (int w = 1; w < nch; ++w) {
                                    gv += sm.red[w][tid];
                                    uv += sm.red[w][16 * GT + tid];
                                }
                                const float inv = norm_scale();
                                gv = inv * gv;
                                uv = inv * uv;
                                v = gv * (uv / (1.0f + expf(-gv)));
                            }
                            put_split(&sm.dp[0][0], split_stride(32), tid, v);
                        }
                    }
                    bar();
                    mark(s, 16 * l + 11);
                    // Down partials on the matrix cores: tiles wave + 8 m of
                    // the H rows, one K-step over the block's 32 columns;
                    // each row stored as owner r / 8's partial of block f
                    // (two rows per store).
                    {
                        const u32x4 da = a_frag(&sm.dp[0][0], a_offset(split_stride(32)), 0);
                        const int nbd = A()->nbd;
                        uint64_t *pdown = A()->pdown;
                        f32x4 acc[ND];
#pragma unroll
                        for (int m = 0; m < ND; ++m) acc[m] = mfma_bf16(da, W[NG + m], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int m = 0; m < ND; ++m)
                            store_tile(tile_dot(acc[m]), (wave + kWaves * m) * 16, H, tD,
                                       [&](int r) { return pdown + ((size_t)(r / kOwn) * nbd + f) * kOwn + r % kOwn; });
                    }
                    mark(s, 16 * l + 12);
                }

                // ---- Owners: the down partials of their rows summed in block
                // order (lane j adds blocks j, j + 64, ...; then the fixed
                // wave tree), + residual.
                if (isOwner()) {
                    const int nbd = A()->nbd;
                    gather(tb, A()->pdown + (size_t)fIdx() * nbd * kOwn, nbd * kOwn, tD, A()->abort_flag);
                    bar();
                    mark(s, 16 * l + 13);
                    float v = 0.f;
                    for (int j = lane_here(); j < nbd; j += 64) v += val_of(tb[j * kOwn + wave]);
                    v = wave_sum(v);
                    if (ownRow() < H) {
                        h_own = h_own + v;
                        if (lane_here() == 0) sm.out[wave] = h_own;
                    }
                    bar();
                    const int cnt = min(kOwn, H - fIdx() * kOwn);
                    if (wave == kDmaWave && lane_here() < cnt)
                        stf(A()->hid1 + fIdx() * kOwn + lane_here(), sm.out[lane_here()], tE);
                    mark(s, 16 * l + 14);
                }
            }
            lm_head(s);
            ++pos;
        }
    }
    // Loads still in flight (refills that read nothing) retire before the
    // waves end.
    wait_vm();
}

struct Variant {
    int hd, g, uh, ks, otw, gt;
};

// Shapes with a built kernel: Qwen2-0.5B (hidden 896, 14/2 heads of 64,
// intermediate 4864) and the two small test shapes.
constexpr Variant kVariants[] = {
    {64, 7, 2, 28, 7, 2},
    {64, 2, 1, 4, 1, 1},
    {128, 4, 1, 8, 2, 1},
};

int units_per_lane(int cols, int elems_per_unit) { return (cols / elems_per_unit + 63) / 64; }

// The block slot of each q head within a run (FusedArgs::slot_head): the
// heads of one KV group on their own XCDs (group g on XCDs g * 8 / kv_heads
// onward, head i of the group on XCD i % (8 / kv_heads) of those, in slot
// layer i / (8 / kv_heads)) where the group count divides the XCD count and
// the slots allow; else head h in slot h.
void item_slots(int q_heads, int kv_heads, int32_t (&slot_head)[64]) {
    for (int32_t &v : slot_head) v = -1;
    const int qp = heads_padded(q_heads), layers = qp / kXcds;
    const int G = kv_heads > 0 ? q_heads / kv_heads : 0;
    const int xpg = kv_heads > 0 && kv_heads <= kXcds && kXcds % kv_heads == 0 ? kXcds / kv_heads : 0;
    if (qp <= 64 && xpg > 0 && G * kv_heads == q_heads && (G + xpg - 1) / xpg <= layers) {
        // Head i of group g: XCD g xpg + i % xpg, slot layer i / xpg.
        for (int h = 0; h < q_heads; ++h) {
            const int g = h / G, i = h % G;
            slot_head[(i / xpg) * kXcds + g * xpg + i % xpg] = h;
        }
        return;
    }
    for (int h = 0; h < q_heads && h < 64; ++h) slot_head[h] = h;
}

FusedGeom geometry(int H, int q_heads, int kv_heads, int hd, int I, bool kv_f32, int blocks) {
    FusedGeom g{};
    g.nf = blocks * 5 / 8;
    // FFN blocks of exactly 32 gate/up rows where that many still fit and
    // cover the owners: the down columns then fill one matrix-core K-step
    // with no zero padding (Qwen2-0.5B: 152 blocks instead of 160 x 31 rows).
    const int n32 = (I + 31) / 32;
    if (n32 <= g.nf && n32 >= H / kOwn) g.nf = n32;
    g.f0 = blocks - g.nf;
    g.nkv = (kv_heads * hd + kWaves - 1) / kWaves;  // one rotation pair of K/V rows per wave
    g.kv0 = g.f0 - g.nkv;
    g.s_cap = q_heads > 0 ? std::min(kMaxSplits, g.kv0 / heads_padded(q_heads)) : 0;
    const int row = hd * (kv_f32 ? 4 : 2);
    g.ip_max = 0;
    for (int ip = TP; ip <= kIpMax && 2 * ip * row <= kKvLdsMax; ip *= 2) g.ip_max = ip;
    g.no = H / kOwn;
    g.rb = g.nf > 0 ? fused_gate_rows(I, g.nf) : 0;
    g.rp = g.nf > 0 ? fused_gate_rows_padded(I, g.nf) : 0;
    g.nbd = g.rb > 0 ? (I + g.rb - 1) / g.rb : 0;
    g.ni_max = q_heads * g.s_cap;
    return g;
}

size_t static_lds_bytes(int hd) {
    return sizeof(Shm) + (hd == 64 ? sizeof(ItemShm<64>) : sizeof(ItemShm<128>));
}

const Variant *find_variant(int fmt, int H, int q_heads, int kv_heads, int hd, int I, bool kv_f32, int blocks) {
    if (fmt != FMT_BF16 || kv_heads <= 0 || q_heads % kv_heads || blocks < 64) return nullptr;
    const int g = q_heads / kv_heads, qd = q_heads * hd;
    if (H % 8 || qd % 8 || I % 8 || H > 1024 || q_heads > 64) return nullptr;
    const FusedGeom geo = geometry(H, q_heads, kv_heads, hd, I, kv_f32, blocks);
    // The down product takes a block's gate/up rows as one K-step of 32.
    if (geo.s_cap < 1 || geo.ip_max < TP || geo.no > geo.nf || geo.rp > 32 || geo.kv0 < heads_padded(q_heads)) return nullptr;
    const LdsLayout lay = lds_layout(H, hd, kv_f32 ? 4 : 2, geo.ip_max, geo.ni_max, geo.nbd, blocks);
    if (lay.tbw > kMaxGather || (size_t)lay.total + static_lds_bytes(hd) > device_max_lds()) return nullptr;
    for (const Variant &v : kVariants) {
        if (v.hd != hd || v.g != g) continue;
        // The split input holds exactly KS K-steps (the LDS layout pads H
        // to 32); H rows in OTW tiles per wave; gate rows in GT tiles.
        if (units_per_lane(H, 8) > v.uh || (H + 31) / 32 != v.ks) continue;
        if ((H + 16 * kWaves - 1) / (16 * kWaves) > v.otw || (geo.rb + 15) / 16 > v.gt) continue;
        return &v;
    }
    return nullptr;
}

template <int HD, int G, class KT, int UH, int KS, int OTW, int GT>
int launch_one(FusedArgs a, int nb, hipStream_t s) {
    auto k = decode_flow_kernel<HD, G, KT, UH, KS, OTW, GT>;
    const FusedGeom geo = geometry(a.H, a.q_heads, a.kv_heads, HD, a.I, sizeof(KT) == 4, nb);
    // Positions per item: the shortest run that lets the launch's longest
    // context fit the item blocks.
    int ip = TP;
    while (ip < geo.ip_max && (a.ctx_end + ip - 1) / ip > geo.s_cap) ip *= 2;
    a.splits = (int)((a.ctx_end + ip - 1) / ip);
    if (a.splits > geo.s_cap) return fail("HIP backend: context too long for the persistent decode kernel.");
    a.ip = ip;
    a.ni = a.q_heads * a.splits;
    a.kv0 = geo.kv0;
    a.nkv = geo.nkv;
    a.f0 = geo.f0;
    a.nf = geo.nf;
    a.no = geo.no;
    a.nbd = geo.nbd;
    a.rb = geo.rb;
    a.rp = geo.rp;
    a.head_blocks = std::min(nb, (a.V + kWaves - 1) / kWaves);
    item_slots(a.q_heads, a.kv_heads, a.slot_head);
    const LdsLayout lay = lds_layout(a.H, HD, (int)sizeof(KT), ip, a.ni, a.nbd, nb);
    a.lds_xs = lay.xs;
    a.lds_xb = lay.xb;
    a.lds_q = lay.q;
    a.lds_kv = lay.kv;
    a.lds_emb = lay.emb;
    a.lds_g1 = lay.g1;
    a.lds_g2 = lay.g2;
    a.lds_total = lay.total;
    const size_t lds = (size_t)lay.total;
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
    if (v.hd == 64 && v.g == 7) return launch_one<64, 7, KT, 2, 28, 7, 2>(a, nb, s);
    if (v.hd == 64 && v.g == 2) return launch_one<64, 2, KT, 1, 4, 1, 1>(a, nb, s);
    if (v.hd == 128 && v.g == 4) return launch_one<128, 4, KT, 1, 8, 2, 1>(a, nb, s);
    return fail("HIP backend: no persistent decode kernel for this shape.");
}

}  // namespace

bool fused_decode_supported(int fmt, int H, int q_heads, int kv_heads, int head_dim, int I, bool aligned16,
                            int blocks) {
    // Either KV precision: the LDS check is made for the wider one.
    return aligned16 && blocks > 0 && find_variant(fmt, H, q_heads, kv_heads, head_dim, I, true, blocks) != nullptr;
}

FusedGeom fused_geometry(int H, int q_heads, int kv_heads, int head_dim, int I, bool kv_f32, int blocks) {
    return geometry(H, q_heads, kv_heads, head_dim, I, kv_f32, blocks);
}

// dst[b][r][j] = down[r][b rb + j] for j < rb and b rb + j < I, else 0;
// one thread per element of dst.
__global__ void down_columns_kernel(const uint16_t *down, size_t stride, int H, int I, int rb, int rp, int nf,
                                    uint16_t *dst) {
    const size_t n = (size_t)nf * H * rp;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(t % rp);
        const size_t br = t / rp;
        const int r = (int)(br % H), b = (int)(br / H);
        const long col = (long)b * rb + j;
        dst[t] = j < rb && col < I ? ((const uint16_t *)((const uint8_t *)down + (size_t)r * stride))[col] : (uint16_t)0;
    }
}

int fused_down_columns(const uint16_t *down, size_t stride, int H, int I, int nf, uint16_t *dst, hipStream_t s) {
    const int rb = fused_gate_rows(I, nf), rp = fused_gate_rows_padded(I, nf);
    const size_t n = (size_t)nf * H * rp;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(down_columns_kernel, dim3(grid), dim3(256), 0, s, down, stride, H, I, rb, rp, nf, dst);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int fused_decode_blocks() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

int launch_decode_fused(FusedArgs a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s) {
    const int nb = fused_decode_blocks();
    if (nb <= 0) return fail("HIP backend: cannot size the persistent decode grid.");
    const Variant *v = find_variant(fmt, a.H, a.q_heads, a.kv_heads, head_dim, a.I, kv_f32, nb);
    if (!v || v->g != group) return fail("HIP backend: no persistent decode kernel for this shape.");
    if (kv_f32) return launch_kt<float>(*v, a, nb, s);
    return launch_kt<uint16_t>(*v, a, nb, s);
}

}  // namespace chip
