// Persistent dataflow decode kernel: one cooperative launch (one 512-thread
// block per CU) runs whole decode steps -- embedding, every layer, LM head,
// greedy argmax -- with no device-wide barrier.
//
// Per layer five phases, per step one more:
//   A  QKV rows (fused RMSNorm, bias, RoPE); K/V rows appended to the pages
//   B  GQA attention: one item = (KV head, run of 128 positions, q head) when
//      those items fit the grid, else (KV head, run) with all q heads of the
//      group; two-pass softmax, (output, max, sum) partials per q head
//   C  every o_proj block merges all partials in split order itself, then
//      o_proj + residual
//   D  gate/up (fused RMSNorm) + SwiGLU
//   E  down + residual
//   H  LM head (fused final RMSNorm) + per-block argmax partials; blocks that
//      need the next token reduce all partials themselves (ties to the last
//      index, engine.rs:2247-2253)
//
// Phases are chained through the data. Every value one block hands to
// another is a 64-bit word {f32 bits, tag}, where the tag names the phase
// instance that produced it (launch base + step * (5L + 1) + 5 * layer +
// phase). Aligned 8-byte stores are single-copy atomic, so value and tag
// arrive together, and a consumer knows its inputs are complete when every
// word it copied carries the expected tag.
//
// Roles inside a block. Waves 0-6 (compute waves) own QKV, o_proj and down
// rows; wave 7 (the spare wave) owns only gate/up rows (like every wave) and
// copies the attention item's cached K/V rows and the RMSNorm gains into LDS. Every wave polls: a phase's tagged input
// words are split into 128-word chunks, wave w copies chunks w, w + 8, ...
// into LDS with direct global->LDS loads (16 bytes per lane, device-coherent
// sc1), checks their tags there and re-loads only the stale ones; all waves
// then stage the f32 vector the dots read (RMSNorm fused where the phase has
// one). The waves meet only at LDS barriers that wait on LDS traffic alone
// (s_waitcnt lgkmcnt(0); s_barrier), never on vector memory.
//
// Weight streaming. Weight rows live in registers. A layer's o_proj, gate/up
// and down rows are issued right after its attention phase (the o_proj/down
// blocks idle while QKV and attention run), the next layer's QKV rows right
// after gate/up, and layer 0's after the LM head. Issuing a phase's rows just
// before its dot would stall the dot: a CU holds only so many outstanding
// misses. The loads are buffer loads issued on every path, with rows a wave
// does not own pointed past the buffer's range (those lanes read nothing and
// return 0), so the compiler counts outstanding loads exactly and each use
// waits only for its own rows. The LDS copies and the hand-off stores are
// inline assembly for the same reason: the compiler would otherwise make
// LDS reads and later loads wait for them.
//
// Buffer reuse needs no barrier: a block polls a phase's inputs only in a
// phase where it also produces outputs, and every buffer is rewritten only by
// a phase that transitively depends on all of those outputs. Only blocks
// that own LM-head rows (and so wait for the final hidden state) write
// argmax partials; those alternate between two buffers by step parity.
//
// Every poll is bounded: on timeout a block raises the abort word, which all
// polls watch, so every later poll gives up within a few rounds and the
// launch runs to its end on stale values (no wave leaves early: an exit inside
// the layer loop would add control-flow paths that make the compiler's waits
// for weight rows conservative). The host sees the word, discards the steps
// and resets the tagged words. The only data-dependent address, the token,
// keeps its last good value when its poll gives up.
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
constexpr int kCW = kWaves - 1;        // compute waves 0 .. kCW - 1
constexpr int kSpareWave = kWaves - 1;  // owns no weight rows
constexpr int TP = 64;                 // positions per KV page
constexpr int kItemPos = 2 * TP;       // positions per attention item, at most
// Positions per item for a K/V row size: two pages, or one when a row is
// wider than 256 bytes (one item's K and V rows stay within 64 KB of LDS).
__host__ __device__ constexpr int item_positions(int row_bytes) { return row_bytes <= 256 ? 2 * TP : TP; }
constexpr int kChunk = 128;            // tagged words per wave-wide 16-byte-per-lane load
constexpr int kMaxChunks = 128;        // largest gather: 16384 words
constexpr long kSpinLimit = 1L << 20;
constexpr uint32_t kNoRead = 0x80000000u;  // buffer offset past every range

// The f32 vector the dot products read sits in LDS with every 8 elements
// padded to 10 floats: a lane reads the 8 x values of its 16-byte weight unit
// at a 40-byte stride, so the lanes of a quarter wave hit distinct banks (at
// the unpadded 32-byte stride, lanes 8 apart share banks and seven waves
// reading one vector serialise on the conflicts).
__host__ __device__ constexpr int xpad(int i) { return (i >> 3) * 10 + (i & 7); }

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
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// N device-coherent 16-byte loads p[i] -> r[i] and the wait for all of them in
// one asm statement: no instruction sees r before its load has landed.
template <int N>
__device__ __forceinline__ void poll16(u32x4 (&r)[8], const uint64_t *const (&p)[8]) {
    if constexpr (N == 1)
        asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0])
                     : "v"(p[0])
                     : "memory");
    else if constexpr (N == 2)
        asm volatile("global_load_dwordx4 %0, %2, off sc1\n\tglobal_load_dwordx4 %1, %3, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1])
                     : "v"(p[0]), "v"(p[1])
                     : "memory");
    else if constexpr (N == 3)
        asm volatile("global_load_dwordx4 %0, %3, off sc1\n\tglobal_load_dwordx4 %1, %4, off sc1\n\tglobal_load_dwordx4 %2, %5, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2])
                     : "memory");
    else if constexpr (N == 4)
        asm volatile("global_load_dwordx4 %0, %4, off sc1\n\tglobal_load_dwordx4 %1, %5, off sc1\n\tglobal_load_dwordx4 %2, %6, off sc1\n\tglobal_load_dwordx4 %3, %7, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3])
                     : "memory");
    else if constexpr (N == 5)
        asm volatile("global_load_dwordx4 %0, %5, off sc1\n\tglobal_load_dwordx4 %1, %6, off sc1\n\tglobal_load_dwordx4 %2, %7, off sc1\n\tglobal_load_dwordx4 %3, %8, off sc1\n\tglobal_load_dwordx4 %4, %9, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4])
                     : "memory");
    else if constexpr (N == 6)
        asm volatile("global_load_dwordx4 %0, %6, off sc1\n\tglobal_load_dwordx4 %1, %7, off sc1\n\tglobal_load_dwordx4 %2, %8, off sc1\n\tglobal_load_dwordx4 %3, %9, off sc1\n\tglobal_load_dwordx4 %4, %10, off sc1\n\tglobal_load_dwordx4 %5, %11, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5])
                     : "memory");
    else if constexpr (N == 7)
        asm volatile("global_load_dwordx4 %0, %7, off sc1\n\tglobal_load_dwordx4 %1, %8, off sc1\n\tglobal_load_dwordx4 %2, %9, off sc1\n\tglobal_load_dwordx4 %3, %10, off sc1\n\tglobal_load_dwordx4 %4, %11, off sc1\n\tglobal_load_dwordx4 %5, %12, off sc1\n\tglobal_load_dwordx4 %6, %13, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6])
                     : "memory");
    else if constexpr (N == 8)
        asm volatile("global_load_dwordx4 %0, %8, off sc1\n\tglobal_load_dwordx4 %1, %9, off sc1\n\tglobal_load_dwordx4 %2, %10, off sc1\n\tglobal_load_dwordx4 %3, %11, off sc1\n\tglobal_load_dwordx4 %4, %12, off sc1\n\tglobal_load_dwordx4 %5, %13, off sc1\n\tglobal_load_dwordx4 %6, %14, off sc1\n\tglobal_load_dwordx4 %7, %15, off sc1\n\ts_waitcnt vmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
                     : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7])
                     : "memory");
}

// Both words of a 16-byte unit (value, tag, value, tag) at word w of n carry
// `tag` (words past n count as fresh).
__device__ __forceinline__ bool unit_fresh(u32x4 v, int w, int n, unsigned tag) {
    return (w >= n || v[1] == tag) && (w + 1 >= n || v[3] == tag);
}

// Register form of the gather for a wave that owns N <= 8 chunks: a round
// loads every chunk of the wave into registers and waits for all of them
// (one asm statement), then checks the tags there; once every word is fresh
// the chunks are written to LDS. Re-loading fresh chunks costs traffic but no
// time: a round takes one memory round trip either way, and without the LDS
// round trip of the copy form a round is shorter.
template <int N>
__device__ void gather_regs(uint64_t *dst, const uint64_t *src, int n, unsigned tag, int *abort_flag, int wave,
                            int lane) {
    const uint64_t *p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int w = (wave + kWaves * i) * kChunk + lane * 2;
        p[i] = src + (i < N && w < n ? w : 0);
    }
    long spins = 0;
    while (true) {
        u32x4 r[8];
        poll16<N>(r, p);
        bool stale = false;
#pragma unroll
        for (int i = 0; i < N; ++i) stale |= !unit_fresh(r[i], (wave + kWaves * i) * kChunk + lane * 2, n, tag);
        const bool done = !__any(stale);
        const bool give_up = !done && (++spins > kSpinLimit || ((spins & 15) == 0 && aborted(abort_flag)));
        if (done || give_up) {
            // On a give-up the words are written too, stale or not: they are
            // the source buffer's, so what readers take from them (a token's
            // row index) stays one that buffer held.
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int w = (wave + kWaves * i) * kChunk + lane * 2;
                if (w < n) *(u32x4 *)(dst + w) = r[i];
            }
            if (give_up) raise_abort(abort_flag);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// All waves: copies tagged words src[0, n) into LDS dst[0, n) and waits until
// each carries `tag`. Wave w owns the 128-word chunks w, w + 8, ...; up to
// eight of them it polls in registers (gather_regs), more it loads with direct
// global->LDS copies and re-loads the stale ones until every word of its
// chunks is fresh (its tag reads for eight chunks in flight at a time). The
// caller's barrier then makes all of them visible to the block. A wave's wait
// also covers the weight rows it has in flight. On timeout the abort word is
// raised and the wave moves on with what it has.
__device__ __attribute__((noinline)) void gather(uint64_t *dst, const uint64_t *src, int n, unsigned tag, int *abort_flag) {
    const int lane = lane_here(), wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int chunks = (n + kChunk - 1) / kChunk;
    const int mine = chunks > wave ? (chunks - 1 - wave) / kWaves + 1 : 0;  // at most 16
    switch (mine) {
        case 0: return;
        case 1: return gather_regs<1>(dst, src, n, tag, abort_flag, wave, lane);
        case 2: return gather_regs<2>(dst, src, n, tag, abort_flag, wave, lane);
        case 3: return gather_regs<3>(dst, src, n, tag, abort_flag, wave, lane);
        case 4: return gather_regs<4>(dst, src, n, tag, abort_flag, wave, lane);
        case 5: return gather_regs<5>(dst, src, n, tag, abort_flag, wave, lane);
        case 6: return gather_regs<6>(dst, src, n, tag, abort_flag, wave, lane);
        case 7: return gather_regs<7>(dst, src, n, tag, abort_flag, wave, lane);
        case 8: return gather_regs<8>(dst, src, n, tag, abort_flag, wave, lane);
        default: break;
    }
    const uint32_t *d32 = (const uint32_t *)dst;
    uint32_t pend = (1u << mine) - 1;
    long spins = 0;
    while (pend) {
        const uint32_t issued = pend;
        for (uint32_t m = issued; m; m &= m - 1) {
            const int c = wave + kWaves * __builtin_ctz(m), w = c * kChunk + lane * 2;
            if (w < n) dma16(src + w, dst + c * kChunk);
        }
        wait_vm();
        uint32_t still = 0;
        for (int i0 = 0; i0 < mine; i0 += 8) {
            uint32_t t0[8], t1[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int w = (wave + kWaves * min(i0 + j, mine - 1)) * kChunk + lane * 2;
                t0[j] = d32[2 * w + 1];
                t1[j] = d32[2 * w + 3];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j, w = (wave + kWaves * i) * kChunk + lane * 2;
                const bool stale = (w < n && t0[j] != tag) || (w + 1 < n && t1[j] != tag);
                if (i < mine && ((issued >> i) & 1) && __any(stale)) still |= 1u << i;
            }
        }
        pend = still;
        if (pend) {
            if (++spins > kSpinLimit || ((spins & 15) == 0 && aborted(abort_flag))) {
                raise_abort(abort_flag);
                return;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
}

// Poll wave only: starts copying `bytes` (a multiple of 16) from global
// memory into LDS; completion is awaited with wait_vm.
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
    int token;           // the step's sampled id
    float out[kStage];   // a phase's outputs of the block, stored as one run
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

template <int HD, int G>
struct AttnShm {
    static constexpr int GP = (G + 3) / 4 * 4;
    float p[kItemPos][GP];  // scores, then weights, of position x head
    float red[kWaves][G][HD];
    float m[G], l[G];
};

__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }
__host__ __device__ constexpr int imax(int a, int b) { return a > b ? a : b; }

// Dynamic LDS layout (byte offsets): tagged-word staging, the f32 vector the
// compute waves read (also an attention item's q), one item's K and V rows,
// the merge weights of every (split, q head) and 1 / sum per q head, the
// next step's embedding row and a phase's RMSNorm gains (BF16).
struct LdsLayout {
    int tbw;  // staging words
    int xs, kv, mw, emb, gain, total;
};
__host__ __device__ inline LdsLayout lds_layout(int H, int I, int nq, int hd, int G, int kv_bytes, int blocks,
                                                int max_splits) {
    LdsLayout o{};
    int tbw = imax(imax(H, I), imax((G + 2) * hd, 2 * blocks));
    tbw = imax(tbw, max_splits * nq * (hd + 2));
    const int rb = (I + blocks - 1) / blocks;
    tbw = imax(tbw, (I + rb - 1) / rb * kCW);  // one o/down block's down partials
    o.tbw = round_up(tbw + 2, kChunk);
    const int xf = xpad(imax(imax(H, I), nq * hd)) + 10;
    o.xs = o.tbw * 8;
    o.kv = o.xs + round_up(xf * 4, 16);
    o.mw = o.kv + 2 * item_positions(hd * kv_bytes) * hd * kv_bytes;
    o.emb = o.mw + round_up((max_splits + 1) * nq * 4, 16);
    o.gain = o.emb + round_up(H * 2, 16);
    o.total = o.gain + round_up(H * 2, 16);
    return o;
}

// Poll wave only: starts the copies of the cached K and V rows of positions
// [start, lim) of KV head g into LDS (row p - start of each); completion is
// awaited with wait_vm.
template <int HD, class KT>
__device__ __forceinline__ void load_kv_lds(CArgs *a, uint8_t *k_lds, uint8_t *v_lds, int l, int g, long start,
                                            long lim) {
    constexpr int ROW = HD * (int)sizeof(KT);
    const int lane = lane_here();
    for (long t0 = start; t0 < lim; t0 += TP) {
        const int page = ldc(opaque(a)->page_table, t0 / TP);
        const int bytes = (int)(min((long)TP, lim - t0)) * ROW;
        const size_t off = (((size_t)page * opaque(a)->kv_heads + g) * TP) * ROW;
        const uint8_t *ks = (const uint8_t *)layer_of(a, l)->kc + off, *vs = (const uint8_t *)layer_of(a, l)->vc + off;
        uint8_t *kd = k_lds + (t0 - start) * ROW, *vd = v_lds + (t0 - start) * ROW;
        for (int c = 0; c < bytes; c += 1024) {
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

// One attention item, all waves: q (G heads, f32) in qs, nv K and V rows in
// LDS; writes (unnormalised output, max, sum) per q head of the group to
// part[j * (HD + 2) + ...] (compute waves store, so the poll wave has no
// stores in flight when it polls next).
template <int HD, int G, class KT>
__device__ __forceinline__ void attn_compute(const float *qs, const uint8_t *k_lds, const uint8_t *v_lds, int nv, AttnShm<HD, G> &sh,
                             uint64_t *part, unsigned tag, uint64_t *tr) {
    constexpr int T = HD / 8, P = kThreads / T, ROW = HD * (int)sizeof(KT);
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    const int d8 = tid % T, pg = tid / T;
    auto mark = [&](int ev) {
        if (tr && tid == 0) st_u64(tr + ev, wall_clock64());
    };
    const float scale = 1.0f / sqrtf((float)HD);
    const int passes = (nv + P - 1) / P;
    for (int ps = 0; ps < passes; ++ps) {
        const int pi = ps * P + pg;
        const bool valid = pi < nv;
        float dot[G];
#pragma unroll
        for (int j = 0; j < G; ++j) dot[j] = 0.f;
        if (valid) {
            float kf[8];
            ld8<KT>((const KT *)(k_lds + (size_t)pi * ROW) + d8 * 8, kf);
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
    bar();
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
    bar();
    mark(2);
    // Weighted V: lane owns DPL head dimensions, wave w positions w, w + 8,
    // ...; the waves' sums are added in wave order.
    constexpr int DPL = HD / 64;
    constexpr int GP = AttnShm<HD, G>::GP;
    float acc[G][DPL];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[j][e] = 0.f;
#pragma unroll 4
    for (int pi = wave; pi < nv; pi += kWaves) {
        const KT *vrow = (const KT *)(v_lds + (size_t)pi * ROW) + lane * DPL;
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
        float pj[GP];
#pragma unroll
        for (int j4 = 0; j4 < GP; j4 += 4) {
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
    bar();
    mark(3);
    if (tid < kCW * 64) {
        for (int t = tid; t < G * HD; t += kCW * 64) {
            const int j = t / HD, d = t % HD;
            float o = sh.red[0][j][d];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) o += sh.red[w][j][d];
            stf(part + (size_t)j * (HD + 2) + d, o, tag);
        }
        if (tid < G) {
            stf(part + (size_t)tid * (HD + 2) + HD, sh.m[tid], tag);
            stf(part + (size_t)tid * (HD + 2) + HD + 1, sh.l[tid], tag);
        }
    }
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
// nothing), so the waits count exactly.
template <int UHB>
__device__ __forceinline__ void head_dots(const uint16_t *head, float *logits, const float *xs, int H, int V, int gw,
                                          int W, int head_rows, int &key, uint32_t &idx) {
    constexpr int HB = 4;
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

// UH/UQ: 16-byte units per lane of a row with H / q_heads*HD columns; UP:
// 16-byte units of a down_cols row (one per thread); RGU: gate/up rows per
// wave; UHB: units per lane of a BF16
// head row. Shape values are re-read from the arguments where used (A()) and
// block roles recomputed from them, so that little stays in scalar registers
// across the step loop.
template <int FMT, int HD, int G, class KT, int UH, int UQ, int UP, int RGU, int UHB, bool HS>
__global__ __launch_bounds__(kThreads) void decode_flow_kernel(FusedArgs) {
    using U = Unit<FMT, 16>;
    constexpr int ROW = HD * (int)sizeof(KT);
    // The only read of the kernarg-segment pointer (see opaque()).
    CArgs *const kargs = (CArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    auto A = [kargs]() { return opaque(kargs); };
    auto LY = [kargs](int l) { return layer_of(kargs, l); };
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ Shm sm;
    constexpr int GI = HS ? 1 : G;  // q heads per attention item
    __shared__ AttnShm<HD, GI> ash;
    const int lane = tid_here() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const bool spare = wave == kSpareWave;
    const int b = blockIdx.x;
    uint64_t *tb = (uint64_t *)lds;

    // Roles. o_proj and down rows: blocks [0, nhb), compute wave w of block b
    // owns row kCW * b + w of both (the residual stays in its register). QKV
    // pairs: the next nab blocks (the last ones when the grid is short).
    // Gate/up: every block rb consecutive rows, wave w (the spare wave too)
    // rows w, w + 8, ...
    // Attention items: the last blocks. LM head: every wave of every block.
    auto npairs = [&]() { return (A()->q_heads + 2 * A()->kv_heads) * HD / 2; };
    auto hasA = [&]() {
        const int s0 = A()->a0;
        return b >= s0 && b < s0 + A()->nab;
    };
    auto pairA = [&]() { return (b - A()->a0) * kCW + wave; };
    auto myA = [&]() { return !spare && hasA() && pairA() < npairs(); };
    auto hasH = [&]() { return b < A()->nhb; };
    auto rowH = [&]() { return b * kCW + wave; };
    auto myH = [&]() { return !spare && hasH() && rowH() < A()->H; };
    auto hasD = [&]() { return b * A()->rb < A()->I; };
    auto nrD = [&]() {
        const int rb = A()->rb, I = A()->I;
        int n = 0;
#pragma unroll
        for (int k = 0; k < RGU; ++k) {
            const int j = wave + kWaves * k;
            n += j < rb && b * rb + j < I ? 1 : 0;
        }
        return n;
    };
    auto hasHead = [&]() { return b * kWaves < A()->V; };

    u32x4 wA[2][UH], wC[1][UQ], wD[2 * RGU][UH], wP[2][UP];

    // Weight rows of layer l. Every wave issues the same loads at the same
    // points (the spare wave's and those of rows a wave does not own read
    // nothing), so no path through the loop has a different load count and
    // the compiler's waits stay exact. Issue points: right after B the
    // o_proj, gate/up and down rows of the layer (the o_proj/down blocks are
    // idle while QKV and attention run, and a CU sustains only so many
    // outstanding misses, so issuing later would stall the wave for the
    // transfer), after D the next layer's QKV rows.
    auto load_wA = [&](int l, bool valid) {
        const size_t stride = A()->qkv_stride;
        const int rows = (A()->q_heads + 2 * A()->kv_heads) * HD;
        const Rsrc r = rsrc(LY(l)->qkv, (size_t)rows * stride);
        const bool v = valid && myA();
        const uint32_t off = (uint32_t)(2 * pairA()) * (uint32_t)stride;
        load_row(wA[0], r, off, A()->H / U::E, v);
        load_row(wA[1], r, off + (uint32_t)stride, A()->H / U::E, v);
    };
    auto load_wC = [&](int l, bool valid) {
        const size_t stride = A()->o_stride;
        const Rsrc r = rsrc(LY(l)->o, (size_t)A()->H * stride);
        load_row(wC[0], r, (uint32_t)rowH() * (uint32_t)stride, A()->q_heads * HD / U::E, valid && myH());
    };
    auto load_wD = [&](int l, bool valid) {
        const size_t stride = A()->gu_stride, bytes = (size_t)A()->I * stride;
        const Rsrc rg = rsrc(LY(l)->gate, bytes), ru = rsrc(LY(l)->up, bytes);
        const int n = nrD(), base = b * A()->rb + wave, nH = A()->H / U::E;
#pragma unroll
        for (int k = 0; k < RGU; ++k) {
            const uint32_t off = (uint32_t)(base + kWaves * k) * (uint32_t)stride;
            load_row(wD[2 * k], rg, off, nH, valid && k < n);
            load_row(wD[2 * k + 1], ru, off, nH, valid && k < n);
        }
    };
    // This block's down_cols rows: output rows q and q + 512 of thread q,
    // UP units each (units past the padded row read nothing).
    auto load_wP = [&](int l, bool valid) {
        const int H = A()->H;
        const uint32_t row_bytes = (uint32_t)A()->rp * 2u;
        const Rsrc r = rsrc(LY(l)->down_cols, (size_t)gridDim.x * H * row_bytes);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = tid_here() + kThreads * i;
            const bool v = valid && hasD() && row < H;
            const uint32_t base = ((uint32_t)b * (uint32_t)H + (uint32_t)row) * row_bytes;
#pragma unroll
            for (int u = 0; u < UP; ++u) {
                const uint32_t off = v && (uint32_t)u * 16u < row_bytes ? base + (uint32_t)u * 16u : kNoRead;
                wP[i][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
            }
        }
    };

    // Layer 0's inputs need the token: the embedding row (spare wave of QKV
    // blocks, into LDS) and the residual element (compute waves of o/down
    // blocks).
    float h_own = 0.f, emb_r = 0.f;
    auto fetch_embed = [&](int tok) {
        if (spare && hasA()) dma_bytes(lds + A()->lds_emb, A()->embed + (size_t)tok * A()->H, A()->H * 2);
        if (myH()) emb_r = ldc_bf16(A()->embed, (long)tok * A()->H + rowH());
    };
    // A phase's normed input: every wave computes the scale itself (same
    // order, same value) and stages its share of xs.
    auto stage_norm = [&](const void *src, bool bf16_src) {
        const uint16_t *g = (const uint16_t *)(lds + A()->lds_gain);
        float *xs = (float *)(lds + A()->lds_xs);
        const int H = A()->H;
        if (bf16_src) block_stage<true>(xs, src, H, g, wave_norm_scale<true>(src, H, A()->eps));
        else block_stage<false>(xs, src, H, g, wave_norm_scale<false>(src, H, A()->eps));
    };

    int token = __builtin_amdgcn_readfirstlane(__hip_atomic_load(A()->step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    long pos = __builtin_amdgcn_readfirstlane(__hip_atomic_load(A()->step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    load_wA(0, true);
    fetch_embed(token);

    // A block is paced when it waited on the previous step's last layer (or
    // this is the launch's first step): only then are the cached K/V rows of
    // every earlier position written when it starts a step. Blocks with no
    // role in the previous step may run ahead and must not prefetch them.
    bool item_prev = false;
    for (int s = 0; s < A()->steps; ++s, ++pos) {
        const int L = A()->L;
        // Optional per-phase timestamps of one step (thread 0 of each block).
        const bool traced = A()->trace && s == A()->trace_step;
        auto mark = [&](int ev) {
            if (traced && tid_here() == 0) st_u64(A()->trace + (size_t)b * (16 * A()->L + 3) + ev, wall_clock64());
        };
        const unsigned tb0 = A()->tag0 + (unsigned)(s * fused_phases_per_step(L));
        // This block's attention item: KV head ig, positions [kv_start, kv_end).
        const long ctx = pos + 1;
        constexpr int IP = item_positions(ROW);
        const int S = (int)((ctx + IP - 1) / IP);
        // With HS every q head of a group is an item of its own:
        // it = (ig * S + isplit) * G + ih; otherwise it = ig * S + isplit.
        const int it = (int)gridDim.x - 1 - b;
        const bool hasB = it < A()->kv_heads * S * (G / GI);
        const int ih = HS ? it % G : 0;
        int ig = 0, isplit = HS ? it / G : it;  // by subtraction (scalar)
        while (hasB && isplit >= S) {
            isplit -= S;
            ++ig;
        }
        const bool paced = s == 0 || hasA() || hasH() || hasD() || hasHead() || item_prev;
        item_prev = hasB;
        const long kv_start = (long)isplit * IP;
        const long kv_end = min(kv_start + IP, ctx);
        const long kv_lim = min(kv_end, pos);  // cached rows; the new one comes tagged
        const int nv = (int)(kv_end - kv_start);

        for (int l = 0; l < L; ++l) {
            const bool more = l + 1 < L;
            const int ln = more ? l + 1 : l;
            const unsigned tA = tb0 + 5 * l, tB = tA + 1, tC = tA + 2, tD = tA + 3, tE = tA + 4;
            mark(16 * l);
            uint8_t *k_lds = lds + A()->lds_kv, *v_lds = k_lds + IP * ROW;
            float *xs = (float *)(lds + A()->lds_xs);

            // The attention item's cached rows start loading at once (spare
            // wave: no weight rows in flight).
            const bool kv_early = hasB && (l > 0 || paced);
            if (spare && kv_early) load_kv_lds<HD, KT>(kargs, k_lds, v_lds, l, ig, kv_start, kv_lim);

            // ---- A: QKV pairs + RoPE + K/V append. Everything a pair's
            // epilogue reads besides its dot (row scale and bias, rotation
            // factors, page, destinations) is loaded before the input poll:
            // the chain of dependent scalar loads (layer table, pointer,
            // value) would otherwise follow the dot on the critical path.
            bool a_sc = false, a_bias = false, a_rope = false;
            float a_s0 = 0.f, a_s1 = 0.f, a_b0 = 0.f, a_b1 = 0.f, a_c = 0.f, a_sn = 0.f;
            int a_i0 = 0, a_i1 = 0, a_c0 = -1, a_c1 = -1;  // q/K/V word, cache element (bit 30: V)
            if (myA()) {
                const int r0 = 2 * pairA();
                if (const float *sc = LY(l)->qkv_sc) {
                    a_sc = true;
                    a_s0 = ldc(sc, r0);
                    a_s1 = ldc(sc, r0 + 1);
                }
                if (const float *bias = LY(l)->qkv_bias) {
                    a_bias = true;
                    a_b0 = ldc(bias, r0);
                    a_b1 = ldc(bias, r0 + 1);
                }
                const int qd = A()->q_heads * HD, kvd = A()->kv_heads * HD, kvh = A()->kv_heads;
                const int rot = A()->rotary, half = rot / 2;
                const int page = ldc(A()->page_table, pos / TP), slot = (int)(pos % TP);
                if (r0 < qd + kvd) {
                    const bool is_q = r0 < qd;
                    const int base = is_q ? r0 : r0 - qd;
                    const int h = base / HD, d0 = base % HD;
                    int o0 = d0, o1 = d0 + 1;
                    if (d0 < rot) {
                        const int i = d0 / 2;
                        a_rope = true;
                        a_c = ldc(A()->rope_cos, pos * half + i);
                        a_sn = ldc(A()->rope_sin, pos * half + i);
                        o0 = i;
                        o1 = half + i;
                    }
                    if (is_q) {
                        const int q0 = (h / G) * (G + 2) * HD + (h % G) * HD;
                        a_i0 = q0 + o0;
                        a_i1 = q0 + o1;
                    } else {
                        const int k0 = h * (G + 2) * HD + G * HD;
                        a_i0 = k0 + o0;
                        a_i1 = k0 + o1;
                        const int e0 = ((page * kvh + h) * TP + slot) * HD;
                        a_c0 = e0 + o0;
                        a_c1 = e0 + o1;
                    }
                } else {
                    const int base = r0 - qd - kvd;
                    const int h = base / HD, d0 = base % HD;
                    const int v0i = h * (G + 2) * HD + (G + 1) * HD;
                    a_i0 = v0i + d0;
                    a_i1 = v0i + d0 + 1;
                    const int e0 = ((page * kvh + h) * TP + slot) * HD;
                    a_c0 = (e0 + d0) | (1 << 30);
                    a_c1 = (e0 + d0 + 1) | (1 << 30);
                }
                // The values are used here, so their loads complete now,
                // while the block waits for its input anyway.
                asm volatile("" : "+v"(a_s0), "+v"(a_s1), "+v"(a_b0), "+v"(a_b1), "+v"(a_c), "+v"(a_sn));
            }
            if (hasA()) {
                if (spare) dma_bytes(lds + A()->lds_gain, LY(l)->ln1, A()->H * 2);
                if (l > 0) gather(tb, A()->hid1, A()->H, tA - 1, A()->abort_flag);
                if (spare) wait_vm();
                bar();
                if (l == 0) stage_norm(lds + A()->lds_emb, true);
                else stage_norm(tb, false);
                bar();
            }
            mark(16 * l + 1);
            if (myA()) {
                float y[2];
                dot_rows<FMT>(wA, xs, A()->H / U::E, y);
                float v0 = y[0], v1 = y[1];
                if (a_sc) {
                    v0 = v0 * a_s0;
                    v1 = v1 * a_s1;
                }
                if (a_bias) {
                    v0 = v0 + a_b0;
                    v1 = v1 + a_b1;
                }
                if (a_rope) {
                    const float x1 = v0 * a_c - v1 * a_sn, x2 = v1 * a_c + v0 * a_sn;
                    v0 = x1;
                    v1 = x2;
                }
                if (lane == 0) {
                    if (a_c0 >= 0) {
                        KT *cache = (KT *)((a_c0 >> 30) ? LY(l)->vc : LY(l)->kc);
                        st_kv(cache + (a_c0 & ((1 << 30) - 1)), v0);
                        st_kv(cache + (a_c1 & ((1 << 30) - 1)), v1);
                    }
                    uint64_t *qkvn = A()->qkvn;
                    stf(qkvn + a_i0, a_c0 >= 0 ? kv_round<KT>(v0) : v0, tA);
                    stf(qkvn + a_i1, a_c1 >= 0 ? kv_round<KT>(v1) : v1, tA);
                }
            }
            mark(16 * l + 2);

            // ---- B: attention item.
            if (hasB) {
                gather(tb, A()->qkvn + (size_t)ig * (G + 2) * HD, (G + 2) * HD, tA, A()->abort_flag);
                if (!kv_early) {
                    // Not paced: the cached rows are read only once the
                    // block holds q (whose tags prove every earlier position
                    // of this layer written); the spare wave owns no chunk of
                    // the gather, so it waits at a barrier first.
                    bar();
                    if (spare) load_kv_lds<HD, KT>(kargs, k_lds, v_lds, l, ig, kv_start, kv_lim);
                }
                if (spare) wait_vm();
                bar();
                // q (the item's heads) as f32; the new position's K and V rows
                // as stored in the cache.
                for (int i = tid_here(); i < GI * HD; i += kThreads) xs[i] = val_of(tb[ih * HD + i]);
                if (kv_end == ctx)
                    for (int i = tid_here(); i < 2 * HD; i += kThreads) {
                        const float v = val_of(tb[G * HD + i]);
                        KT *row = (KT *)((i < HD ? k_lds : v_lds) + (size_t)(nv - 1) * ROW);
                        if constexpr (sizeof(KT) == 2) row[i % HD] = f32_bf16_rne(v);
                        else row[i % HD] = v;
                    }
                bar();
                mark(16 * l + 3);
                uint64_t *tr = traced ? A()->trace + (size_t)b * (16 * A()->L + 3) + 16 * l + 3 : nullptr;
                attn_compute<HD, GI, KT>(
                    xs, k_lds, v_lds, nv, ash,
                    A()->part + ((size_t)isplit * A()->q_heads + (size_t)ig * G + ih) * (HD + 2), tB, tr);
            }
            // Attention blocks issue these after their item: rows in flight
            // would hold back the item's q poll.
            load_wC(l, true);
            load_wD(l, true);
            load_wP(l, true);
            mark(16 * l + 7);

            // ---- C: partials merged in split order (weights exp(m_s - M),
            // sum L = sum_s w_s l_s), o_proj + residual. Wave w merges q
            // heads w, w + 8, ...: lane s holds split s's max and sum, lanes
            // hold head dimensions for the weighted sum.
            if (hasH()) {
                const int Q = A()->q_heads;
                gather(tb, A()->part, S * Q * (HD + 2), tB, A()->abort_flag);
                bar();
                for (int h = wave; h < Q; h += kWaves) {
                    const uint64_t *ph = tb + (size_t)h * (HD + 2);
                    const size_t stride = (size_t)Q * (HD + 2);
                    const float ms = lane < S ? val_of(ph[lane * stride + HD]) : -INFINITY;
                    const float M = wave_max(ms);
                    const float ws = lane < S ? expf(ms - M) : 0.f;
                    const float lsum = lane < S ? val_of(ph[lane * stride + HD + 1]) : 0.f;
                    float Ls = 0.f;
                    for (int s2 = 0; s2 < S; ++s2) Ls = fmaf(lane_read(ws, s2), lane_read(lsum, s2), Ls);
                    const float linv = 1.0f / Ls;
#pragma unroll
                    for (int e = 0; e < HD / 64; ++e) {
                        const int d = lane + 64 * e;
                        float o = 0.f;
                        for (int s2 = 0; s2 < S; ++s2) o = fmaf(lane_read(ws, s2), val_of(ph[s2 * stride + d]), o);
                        xs[xpad(h * HD + d)] = o * linv;
                    }
                }
                bar();
            }
            mark(16 * l + 8);
            if (myH()) {
                const int r = rowH();
                float y[1];
                dot_rows<FMT>(wC, xs, A()->q_heads * HD / U::E, y);
                mark(16 * l + 14);
                float v = y[0];
                if (const float *sc = LY(l)->o_sc) v = v * ldc(sc, r);
                if (const float *bias = LY(l)->o_bias) v = v + ldc(bias, r);
                const float old = l == 0 ? emb_r : h_own;
                h_own = old + v;
                if (lane == 0) sm.out[wave] = h_own;
            }
            // The block's rows leave as one coalesced run (one writer per
            // line instead of one per wave).
            if (hasH()) {
                bar();
                const int cnt = min(kCW, A()->H - b * kCW);
                if (wave == 0 && lane < cnt) stf(A()->hid0 + b * kCW + lane, sm.out[lane], tC);
            }
            mark(16 * l + 9);

            // ---- D: gate/up + SwiGLU.
            if (hasD()) {
                if (spare) dma_bytes(lds + A()->lds_gain, LY(l)->ln2, A()->H * 2);
                gather(tb, A()->hid0, A()->H, tC, A()->abort_flag);
                if (spare) wait_vm();
                bar();
                stage_norm(tb, false);
                bar();
            }
            mark(16 * l + 10);
            {
                const int n = nrD();
                if (n > 0) {
                    float y[2 * RGU];
                    dot_rows<FMT>(wD, xs, A()->H / U::E, y);
                    const int base = b * A()->rb + wave;
#pragma unroll
                    for (int k = 0; k < RGU; ++k)
                        if (k < n) {
                            const int r = base + kWaves * k;
                            float gv = y[2 * k], uv = y[2 * k + 1];
                            if (const float *gs = LY(l)->gate_sc) {
                                gv = gv * ldc(gs, r);
                                uv = uv * ldc(LY(l)->up_sc, r);
                            }
                            if (lane == 0) sm.out[r - b * A()->rb] = gv * (uv / (1.0f + expf(-gv)));
                        }
                }
                // Zeros after the block's outputs, up to the padded row.
                {
                    const int cnt = hasD() ? min(A()->rb, A()->I - b * A()->rb) : 0;
                    if (tid_here() >= cnt && tid_here() < UP * 8) sm.out[tid_here()] = 0.f;
                }
            }
            // The block's down partials: thread q's output rows r = q, q + 512
            // sum down[r][b rb + j] * act_j over the block's gate/up rows j
            // in order (padding columns and outputs are zero). Every block
            // runs the multiply-adds, so every path consumes the loaded rows
            // (pinned here: the compiler then waits for them once, up front).
            if (hasD()) bar();
            pin(wP);
            {
                const int cnt = hasD() ? min(A()->rb, A()->I - b * A()->rb) : 0;
                float acc[2] = {0.f, 0.f};
#pragma unroll
                for (int u = 0; u < UP; ++u) {
                    float av[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) av[e] = sm.out[8 * u + e];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t raw[4] = {wP[i][u][0], wP[i][u][1], wP[i][u][2], wP[i][u][3]};
                        U::decode(raw, [&](int e, float v) { acc[i] = fmaf(v, av[e], acc[i]); });
                    }
                }
                // Rows up to 7 nhb (the last o/down block's group is whole;
                // rows past H carry zeros).
                if (cnt > 0) {
                    const int rows = A()->nhb * kCW, nbd = A()->nbd;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const int row = tid_here() + kThreads * i;
                        if (row < rows) stf(A()->pdown + ((size_t)(row / kCW) * nbd + b) * kCW + row % kCW, acc[i], tD);
                    }
                }
            }
            load_wA(ln, more);
            mark(16 * l + 11);

            // ---- E: the down partials of this block's rows summed in block
            // order (lane j adds blocks j, j + 64, ...; then the fixed wave
            // tree), + residual. (BF16 weights only: no row scale.)
            uint64_t *hid1 = A()->hid1;
            if (hasH()) {
                const int nbd = A()->nbd;
                gather(tb, A()->pdown + (size_t)b * nbd * kCW, nbd * kCW, tD, A()->abort_flag);
                bar();
            }
            mark(16 * l + 12);
            if (myH()) {
                const int nbd = A()->nbd;
                float v = 0.f;
                for (int j = lane; j < nbd; j += 64) v += val_of(tb[j * kCW + wave]);
                v = wave_sum(v);
                mark(16 * l + 15);
                h_own = h_own + v;
                if (lane == 0) sm.out[wave] = h_own;
            }
            if (hasH()) {
                bar();
                const int cnt = min(kCW, A()->H - b * kCW);
                if (wave == 0 && lane < cnt) stf(hid1 + b * kCW + lane, sm.out[lane], tE);
            }
            mark(16 * l + 13);
        }

        // ---- LM head (BF16, final norm fused) + argmax partials. The weight
        // registers hold the last layer's no-op prefetches; pinned across the
        // head, its row buffers live elsewhere, and no path from a head load
        // reaches a layer's use of a weight register.
        pin(wA);
        pin(wC);
        pin(wD);
        pin(wP);
        const unsigned tH = tb0 + 5 * L;
        int key = INT_MIN;
        uint32_t idx = 0;
        if (hasHead()) {
            if (spare) dma_bytes(lds + A()->lds_gain, A()->final_norm, A()->H * 2);
            gather(tb, A()->hid1, A()->H, tH - 1, A()->abort_flag);
            if (spare) wait_vm();
            bar();
            stage_norm(tb, false);
            bar();
            mark(16 * L);
            const int W = (int)gridDim.x * kWaves, gw0 = b * kWaves + wave, V = A()->V;
            const int head_rows = gw0 < V ? (V - 1 - gw0) / W + 1 : 0;
            head_dots<UHB>(A()->head, A()->logits, (const float *)(lds + A()->lds_xs), A()->H, V, gw0, W, head_rows,
                           key, idx);
        }
        block_best(key, idx, sm);
        pin(wA);
        pin(wC);
        pin(wD);
        pin(wP);
        mark(16 * L + 1);
        uint64_t *am = A()->am + (size_t)(s & 1) * gridDim.x * 2;
        if (hasHead() && tid_here() == 0) {
            stt(am + 2 * b, (uint32_t)key, tH);
            stt(am + 2 * b + 1, idx, tH);
        }
        const bool next = s + 1 < A()->steps;
        load_wA(0, next);
        // Blocks that use the token (embedding row, residual) reduce the
        // partials of every head block. A partial that never arrived (the
        // poll gave up) still holds a valid row index.
        if (hasA() || hasH()) {
            const int head_blocks = A()->head_blocks;
            gather(tb, am, 2 * head_blocks, tH, A()->abort_flag);
            bar();
            if (wave == 0) {
                key = INT_MIN;
                idx = 0;
                for (int i = lane; i < head_blocks; i += 64)
                    better(key, idx, (int)(uint32_t)tb[2 * i], (uint32_t)tb[2 * i + 1]);
                wave_best(key, idx);
                // A row index outside the vocabulary can only come from a
                // poll that gave up; the token then keeps its last value.
                if (lane == 0) sm.token = idx < (uint32_t)A()->V ? (int)idx : token;
            }
            bar();
            token = __builtin_amdgcn_readfirstlane(sm.token);
            if (b == 0 && tid_here() == 0) {
                if (pos + 1 < A()->hist_cap) st_u32(A()->hist + pos + 1, (uint32_t)token);
                st_u32(A()->step, (uint32_t)token);
                st_u32(A()->step + 1, (uint32_t)(pos + 1));
            }
            if (next) fetch_embed(token);
        }
        mark(16 * L + 2);
    }
}

struct Variant {
    int fmt, hd, g, uh, uq, up, rgu, uhb;
};

// Shapes with a built kernel: Qwen2-0.5B (hidden 896, 14/2 heads of 64,
// intermediate 4864) and the two small test shapes.
constexpr Variant kVariants[] = {
    {FMT_BF16, 64, 7, 2, 2, 3, 3, 2},
    {FMT_BF16, 64, 2, 1, 1, 1, 1, 1},
    {FMT_BF16, 128, 4, 1, 2, 1, 1, 1},
};

int units_per_lane(int cols, int elems_per_unit) { return (cols / elems_per_unit + 63) / 64; }

const Variant *find_variant(int fmt, int H, int q_heads, int kv_heads, int hd, int I, int blocks) {
    if (kv_heads <= 0 || q_heads % kv_heads) return nullptr;
    const int g = q_heads / kv_heads, E = fmt == FMT_Q8 ? 16 : 8, W = blocks * kCW;
    const int qd = q_heads * hd, kvd = kv_heads * hd;
    if (H % 8 || qd % E || H % E || I % E) return nullptr;
    if (H > kMaxChunks * kChunk || I > kMaxChunks * kChunk) return nullptr;  // one gather each
    if ((qd + 2 * kvd) / 2 > W || H > W) return nullptr;
    for (const Variant &v : kVariants) {
        if (v.fmt != fmt || v.hd != hd || v.g != g) continue;
        if (units_per_lane(H, E) > v.uh || units_per_lane(qd, E) > v.uq) continue;
        // One thread per down_cols row pair: 7 ceil(H / 7) <= 2 * 512; UP
        // units per row.
        if ((H + kCW - 1) / kCW * kCW > 2 * kThreads || fused_gate_rows_padded(I, blocks) / 8 > v.up) continue;
        const int rb = (I + blocks - 1) / blocks;
        if ((rb + kWaves - 1) / kWaves > v.rgu || rb > kStage || units_per_lane(H, 8) > v.uhb) continue;
        return &v;
    }
    return nullptr;
}

size_t static_lds_bytes(int hd, int g) {
    size_t att = 0;
    if (hd == 64 && g == 7) att = sizeof(AttnShm<64, 7>);
    else if (hd == 64 && g == 2) att = sizeof(AttnShm<64, 2>);
    else if (hd == 128 && g == 4) att = sizeof(AttnShm<128, 4>);
    return sizeof(Shm) + att;
}

template <int FMT, int HD, int G, class KT, int UH, int UQ, int UP, int RGU, int UHB, bool HS>
int launch_one(FusedArgs a, int nb, hipStream_t s) {
    auto k = decode_flow_kernel<FMT, HD, G, KT, UH, UQ, UP, RGU, UHB, HS>;
    const LdsLayout lay = lds_layout(a.H, a.I, a.q_heads, HD, G, (int)sizeof(KT), nb, a.max_splits);
    a.lds_xs = lay.xs;
    a.lds_kv = lay.kv;
    a.lds_mw = lay.mw;
    a.lds_emb = lay.emb;
    a.lds_gain = lay.gain;
    a.lds_total = lay.total;
    const int npairs = (a.q_heads + 2 * a.kv_heads) * HD / 2;
    a.nhb = (a.H + kCW - 1) / kCW;
    a.nab = (npairs + kCW - 1) / kCW;
    a.a0 = a.nhb + a.nab <= nb ? a.nhb : nb - a.nab;
    a.rb = fused_gate_rows(a.I, nb);
    a.rp = fused_gate_rows_padded(a.I, nb);
    a.nbd = (a.I + a.rb - 1) / a.rb;
    a.head_blocks = std::min(nb, (a.V + kWaves - 1) / kWaves);
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

template <class KT, bool HS>
int launch_kt(const Variant &v, const FusedArgs &a, int nb, hipStream_t s) {
    if (v.hd == 64 && v.g == 7) return launch_one<FMT_BF16, 64, 7, KT, 2, 2, 3, 3, 2, HS>(a, nb, s);
    if (v.hd == 64 && v.g == 2) return launch_one<FMT_BF16, 64, 2, KT, 1, 1, 1, 1, 1, HS>(a, nb, s);
    if (v.hd == 128 && v.g == 4) return launch_one<FMT_BF16, 128, 4, KT, 1, 2, 1, 1, 1, HS>(a, nb, s);
    return fail("HIP backend: no persistent decode kernel for this shape.");
}

// Attention items one per (KV head, split, q head) when they all fit the
// grid at the launch's longest context (CHEETAH_HIP_FUSED_HEAD_SPLIT=0: one
// per (KV head, split), all q heads of the group).
bool head_split(const FusedArgs &a, int group, int head_dim, bool kv_f32, int nb) {
    const char *e = getenv("CHEETAH_HIP_FUSED_HEAD_SPLIT");
    if (e && e[0] == '0') return false;
    const long ip = item_positions(head_dim * (kv_f32 ? 4 : 2));
    const long S = (a.ctx_end + ip - 1) / ip;
    return group > 1 && (long)a.kv_heads * S * group <= (long)nb;
}

}  // namespace

int fused_positions_per_item(int head_dim, bool kv_f32) {
    return item_positions(head_dim * (kv_f32 ? 4 : 2));
}

bool fused_decode_supported(int fmt, int H, int q_heads, int kv_heads, int head_dim, int I, bool aligned16,
                            int blocks) {
    return aligned16 && blocks > 0 && find_variant(fmt, H, q_heads, kv_heads, head_dim, I, blocks) != nullptr;
}

// dst[b][r][j] = down[r][b rb + j] for j < rb and b rb + j < I, else 0;
// one thread per element of dst.
__global__ void down_columns_kernel(const uint16_t *down, size_t stride, int H, int I, int rb, int rp, int blocks,
                                    uint16_t *dst) {
    const size_t n = (size_t)blocks * H * rp;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(t % rp);
        const size_t br = t / rp;
        const int r = (int)(br % H), b = (int)(br / H);
        const long col = (long)b * rb + j;
        dst[t] = j < rb && col < I ? ((const uint16_t *)((const uint8_t *)down + (size_t)r * stride))[col] : (uint16_t)0;
    }
}

int fused_down_columns(const uint16_t *down, size_t stride, int H, int I, int blocks, uint16_t *dst, hipStream_t s) {
    const int rb = fused_gate_rows(I, blocks), rp = fused_gate_rows_padded(I, blocks);
    const size_t n = (size_t)blocks * H * rp;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(down_columns_kernel, dim3(grid), dim3(256), 0, s, down, stride, H, I, rb, rp, blocks, dst);
    CHIP_CHECK(hipGetLastError());
    return 0;
}

int fused_decode_blocks() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

int fused_max_splits(int H, int q_heads, int kv_heads, int head_dim, int I, bool kv_f32, int blocks,
                     size_t capacity) {
    // The most splits whose partials every o_proj block can hold in LDS next
    // to everything else (capped by the grid and by `capacity` positions).
    const int kvb = kv_f32 ? 4 : 2, G = q_heads / kv_heads;
    const size_t budget = device_max_lds(), fixed = static_lds_bytes(head_dim, G);
    const size_t per_item = (size_t)item_positions(head_dim * kvb);
    const size_t need = (capacity + per_item - 1) / per_item;
    // At most 64: the merge holds one split per lane.
    int ms = (int)std::min({(size_t)(blocks / kv_heads), std::max<size_t>(need, 1), (size_t)64});
    for (; ms >= 1; --ms) {
        const LdsLayout lay = lds_layout(H, I, q_heads, head_dim, G, kvb, blocks, ms);
        if (fixed + (size_t)lay.total <= budget && lay.tbw <= kMaxChunks * kChunk) return ms;
    }
    return 0;  // not even one split fits: no persistent kernel for this shape
}

int launch_decode_fused(FusedArgs a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s) {
    const int nb = fused_decode_blocks();
    if (nb <= 0) return fail("HIP backend: cannot size the persistent decode grid.");
    const Variant *v = find_variant(fmt, a.H, a.q_heads, a.kv_heads, head_dim, a.I, nb);
    if (!v || v->g != group) return fail("HIP backend: no persistent decode kernel for this shape.");
    const bool hs = head_split(a, group, head_dim, kv_f32, nb);
    if (kv_f32) return hs ? launch_kt<float, true>(*v, a, nb, s) : launch_kt<float, false>(*v, a, nb, s);
    return hs ? launch_kt<uint16_t, true>(*v, a, nb, s) : launch_kt<uint16_t, false>(*v, a, nb, s);
}

}  // namespace chip
