// Persistent decode kernel: one cooperative launch runs whole decode steps
// (embedding, every layer, LM head, greedy argmax) with device-wide barriers
// between the dependent phases instead of kernel boundaries:
//
//   per layer  A  QKV GEMV (fused RMSNorm, bias) + RoPE + KV page append
//              B  GQA attention over the paged cache, split over positions;
//                 the last split to arrive for a KV head merges it
//              C  o_proj GEMV + residual
//              D  gate/up GEMV (fused RMSNorm) + SwiGLU
//              E  down GEMV + residual
//   per step   LM head GEMV (fused final RMSNorm) + per-wave argmax partials;
//              every block then reduces the partials itself (ties to the
//              last index, engine.rs:2247-2253) and starts the next step.
//
// Math per phase is that of the multi-kernel path (gemv.hip, attention.hip,
// misc.hip), which follows the reference path in ops.rs / qwen2.rs.
//
// Cross-block data (hidden, q, K/V rows, attention partials and output, act,
// argmax partials) is written and read with device-scope relaxed atomics,
// i.e. sc1 loads and stores that stay coherent across the XCDs' separate L2
// caches, so no barrier needs an L2 writeback or invalidate. A barrier is:
// every thread waits for its own stores (s_waitcnt), block 0 gathers one
// arrival word per block, then publishes a release word. Every spin is
// bounded: on timeout the kernel raises an abort word that all spins watch,
// and every wave exits. Weights and older KV pages are only read, so they
// use ordinary (non-temporal) loads.
#include "decode_fused.hpp"
#include "wunit.hpp"

namespace chip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int TP = 64;
constexpr long kSpinLimit = 1L << 22;

__device__ __forceinline__ float ld1(const float *p) {
    return __uint_as_float(__hip_atomic_load((const unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st1(float *p, float v) {
    __hip_atomic_store((unsigned *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ldu(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stu(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_kv(uint16_t *p, float v) {
    __hip_atomic_store(p, f32_bf16_rne(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_kv(float *p, float v) { st1(p, v); }

// Eight consecutive K/V elements, device-coherent loads.
__device__ __forceinline__ void ld8(const uint16_t *p, float (&f)[8]) {
    const unsigned long long a = __hip_atomic_load((const unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long b = __hip_atomic_load((const unsigned long long *)(p + 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t w0 = (uint32_t)a, w1 = (uint32_t)(a >> 32), w2 = (uint32_t)b, w3 = (uint32_t)(b >> 32);
    f[0] = bf16_lo(w0); f[1] = bf16_hi(w0); f[2] = bf16_lo(w1); f[3] = bf16_hi(w1);
    f[4] = bf16_lo(w2); f[5] = bf16_hi(w2); f[6] = bf16_lo(w3); f[7] = bf16_hi(w3);
}
__device__ __forceinline__ void ld8(const float *p, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const unsigned long long a = __hip_atomic_load((const unsigned long long *)(p + i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        f[i] = __uint_as_float((uint32_t)a);
        f[i + 1] = __uint_as_float((uint32_t)(a >> 32));
    }
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

struct Shm {
    float red[kWaves];
    int flag;
    int ikey[kWaves];
    uint32_t iidx[kWaves];
};

// Device-wide barrier (see the file comment). Returns false when the kernel
// must stop (a spin timed out here or elsewhere).
__device__ bool grid_sync(const FusedArgs &a, unsigned epoch, Shm &sm) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int tid = threadIdx.x;
    if (blockIdx.x == 0) {
        int ok = 1;
        for (int b = tid + 1; b < (int)gridDim.x; b += kThreads) {
            long spins = 0;
            while (ldu(a.arrive + b) < epoch) {
                if (++spins > kSpinLimit || ldu((const unsigned *)a.abort_flag)) {
                    stu((unsigned *)a.abort_flag, 1u);
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (!ok) break;
        }
        if (!ok) sm.flag = 0;
        __syncthreads();
        if (tid == 0) {
            if (sm.flag) stu(a.go, epoch);
            else stu(a.go, 0xFFFFFFFFu);
        }
    } else if (tid == 0) {
        stu(a.arrive + blockIdx.x, epoch);
        long spins = 0;
        unsigned g;
        while ((g = ldu(a.go)) < epoch) {
            if (++spins > kSpinLimit || ldu((const unsigned *)a.abort_flag)) {
                stu((unsigned *)a.abort_flag, 1u);
                sm.flag = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (g == 0xFFFFFFFFu) sm.flag = 0;
    }
    __syncthreads();
    return sm.flag != 0;
}

// x (device-coherent source, or BF16 table row) -> LDS, optionally RMSNorm'd
// exactly as the GEMV prologue does: x * (inv * gain).
template <bool FROM_BF16>
__device__ void stage(float *xs, const void *src, int n, const uint16_t *gain, float eps, Shm &sm) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
    for (int i = tid; i < n; i += kThreads) {
        const float v = FROM_BF16 ? bf16_f32(((const uint16_t *)src)[i]) : ld1((const float *)src + i);
        xs[i] = v;
        ss = fmaf(v, v, ss);
    }
    if (gain) {
        ss = wave_sum(ss);
        if (lane == 0) sm.red[wave] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total += sm.red[w];
        const float inv = 1.0f / sqrtf(total / (float)n + eps);
        for (int i = tid; i < n; i += kThreads) xs[i] = xs[i] * (inv * bf16_f32(gain[i]));
    }
    __syncthreads();
}

// NM row dot products against xs (wave-wide; the sums land in every lane).
template <int FMT, int UB, int NM>
__device__ void wave_dots(const uint8_t *const (&rp)[NM], const float *xs, int K, float (&out)[NM]) {
    using U = Unit<FMT, UB>;
    constexpr int E = U::E, D = U::D;
    constexpr int UNROLL = UB == 16 ? 4 : 8;
    const int lane = threadIdx.x & 63;
    const int n_units = K / E;
    float acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] = 0.f;
    for (int u0 = lane; u0 < n_units; u0 += 64 * UNROLL) {
        uint32_t raw[UNROLL][NM][D];
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) {
            const int u = u0 + 64 * i;
            if (u < n_units)
#pragma unroll
                for (int m = 0; m < NM; ++m) load_raw<UB>(rp[m] + (size_t)u * UB, raw[i][m]);
        }
#pragma unroll
        for (int i = 0; i < UNROLL; ++i) {
            const int u = u0 + 64 * i;
            if (u < n_units) {
                const float *xu = xs + u * E;
#pragma unroll
                for (int m = 0; m < NM; ++m)
                    U::decode(raw[i][m], [&](int e, float wv) { acc[m] = fmaf(wv, xu[e], acc[m]); });
            }
        }
    }
    for (int e = n_units * E + lane; e < K; e += 64) {
        const float xv = xs[e];
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[m] = fmaf(U::element(rp[m], e), xv, acc[m]);
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) out[m] = wave_sum(acc[m]);
}

template <int HD, int G>
struct AttnShm {
    float p[G][TP];
    float alpha[G];
    float red[kWaves][G][HD];
    float l[G];
    float w[G][64];
    float inv[G];
    int last;
};

// One attention item: KV head g, positions [start, end) of ctx, all G heads.
// With one split the output is written normalised; otherwise a partial and
// the last block to arrive for this KV head merges the S partials.
template <int HD, int G, class KT>
__device__ void attn_item(const FusedArgs &a, const FusedLayer &ly, int g, int split, int S, long ctx,
                          AttnShm<HD, G> &sh) {
    constexpr int T = HD / 8, P = kThreads / T, JW = (G + 3) / 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d8 = tid % T, pg = tid / T;
    long chunk = (ctx + S - 1) / S;
    chunk = (chunk + TP - 1) / TP * TP;
    const long start = (long)split * chunk;
    const long end = min(start + chunk, ctx);
    const size_t part_head = (size_t)S * (HD + 2);
    float *part = a.part + (size_t)g * G * part_head + (size_t)split * (HD + 2);
    const float scale = 1.0f / sqrtf((float)HD);
    float m_run[JW], l_run[JW];
#pragma unroll
    for (int i = 0; i < JW; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
    }
    float acc[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    if (start < ctx) {
        float qr[G][8];
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) qr[j][e] = ld1(a.qrot + (size_t)(g * G + j) * HD + d8 * 8 + e);
        for (long t0 = start; t0 < end; t0 += TP) {
            const int page = a.page_table[t0 / a.page_size];
            const size_t tile_off = (((size_t)page * a.kv_heads + g) * a.page_size + t0 % a.page_size) * HD;
            const KT *kt = (const KT *)ly.kc + tile_off;
            const KT *vt = (const KT *)ly.vc + tile_off;
            float vf[TP / P][8];
#pragma unroll
            for (int p = 0; p < TP / P; ++p)
                if (t0 + p * P + pg < end) ld8(vt + (size_t)(p * P + pg) * HD + d8 * 8, vf[p]);
#pragma unroll
            for (int p = 0; p < TP / P; ++p) {
                const int pi = p * P + pg;
                const bool valid = t0 + pi < end;
                float dot[G];
#pragma unroll
                for (int j = 0; j < G; ++j) dot[j] = 0.f;
                if (valid) {
                    float kf[8];
                    ld8(kt + (size_t)pi * HD + d8 * 8, kf);
#pragma unroll
                    for (int j = 0; j < G; ++j)
#pragma unroll
                        for (int e = 0; e < 8; ++e) dot[j] = fmaf(kf[e], qr[j][e], dot[j]);
                }
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const float sum = group_sum<T>(dot[j]);
                    if (d8 == 0) sh.p[j][pi] = valid ? sum * scale : -INFINITY;
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < JW; ++i) {
                const int j = wave + 4 * i;
                if (j < G) {
                    const float sc = sh.p[j][lane];
                    const float m_new = fmaxf(m_run[i], wave_max(sc));
                    const float pv = sc == -INFINITY ? 0.f : expf(sc - m_new);
                    sh.p[j][lane] = pv;
                    const float l_tile = wave_sum(pv);
                    const float alpha = m_run[i] == -INFINITY ? 0.f : expf(m_run[i] - m_new);
                    l_run[i] = l_run[i] * alpha + l_tile;
                    m_run[i] = m_new;
                    if (lane == 0) sh.alpha[j] = alpha;
                }
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float al = sh.alpha[j];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[j][e] *= al;
            }
#pragma unroll
            for (int p = 0; p < TP / P; ++p) {
                const int pi = p * P + pg;
                if (t0 + pi < end) {
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        const float pj = sh.p[j][pi];
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(pj, vf[p][e], acc[j][e]);
                    }
                }
            }
            __syncthreads();
        }
    }
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
            for (int e = 0; e < 8; ++e) sh.red[wave][j][d8 * 8 + e] = acc[j][e];
    }
#pragma unroll
    for (int i = 0; i < JW; ++i) {
        const int j = wave + 4 * i;
        if (j < G && lane == 0) {
            sh.l[j] = l_run[i];
            if (S > 1) {
                st1(part + j * part_head + HD, m_run[i]);
                st1(part + j * part_head + HD + 1, l_run[i]);
            }
        }
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += kThreads) {
        const int j = t / HD, d = t % HD;
        const float o = sh.red[0][j][d] + sh.red[1][j][d] + sh.red[2][j][d] + sh.red[3][j][d];
        if (S == 1) st1(a.attn + (size_t)(g * G + j) * HD + d, o / sh.l[j]);
        else st1(part + j * part_head + d, o);
    }
    if (S == 1) return;
    // Count this split in; the last one merges (split order, deterministic).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(a.attn_count + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = old == (unsigned)(S - 1);
        if (sh.last) stu(a.attn_count + g, 0u);
    }
    __syncthreads();
    if (!sh.last) return;
    const float *pg0 = a.part + (size_t)g * G * part_head;
#pragma unroll
    for (int i = 0; i < JW; ++i) {
        const int j = wave + 4 * i;
        if (j < G) {
            const float *pj = pg0 + (size_t)j * part_head;
            const float m = lane < S ? ld1(pj + (size_t)lane * (HD + 2) + HD) : -INFINITY;
            const float M = wave_max(m);
            const float w = m == -INFINITY ? 0.f : expf(m - M);
            const float l = w != 0.f ? ld1(pj + (size_t)lane * (HD + 2) + HD + 1) : 0.f;
            const float L = wave_sum(w * l);
            if (lane < S) sh.w[j][lane] = w;
            if (lane == 0) sh.inv[j] = 1.0f / L;
        }
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += kThreads) {
        const int j = t / HD, d = t % HD;
        const float *pj = pg0 + (size_t)j * part_head;
        float o = 0.f;
        for (int s = 0; s < S; ++s) {
            const float w = sh.w[j][s];
            if (w != 0.f) o = fmaf(w, ld1(pj + (size_t)s * (HD + 2) + d), o);
        }
        st1(a.attn + (size_t)(g * G + j) * HD + d, o * sh.inv[j]);
    }
}

template <int FMT, int UB, int HD, int G, class KT>
__global__ __launch_bounds__(kThreads) void decode_fused_kernel(FusedArgs a) {
    extern __shared__ float xs[];
    __shared__ Shm sm;
    __shared__ AttnShm<HD, G> ash;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NB = gridDim.x, W = NB * kWaves;
    const int gw = blockIdx.x * kWaves + wave;
    const int H = a.H, qd = a.q_heads * HD, kvd = a.kv_heads * HD;
    const int half = a.rotary / 2;
    if (tid == 0) sm.flag = 1;
    __syncthreads();
    unsigned epoch = ldu(a.epoch_base);
    int token = __hip_atomic_load(a.step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    long pos = __hip_atomic_load(a.step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    for (int step = 0; step < a.steps; ++step, ++pos) {
        const long ctx = pos + 1;
        const int S = (int)max(1L, min((ctx + TP - 1) / TP, (long)a.max_splits));
        const float *cr = a.rope_cos + (size_t)pos * half;
        const float *sr = a.rope_sin + (size_t)pos * half;
        const int page = a.page_table[pos / a.page_size];
        const int slot = (int)(pos % a.page_size);
        const uint16_t *emb = a.embed + (size_t)token * H;
        for (int l = 0; l < a.L; ++l) {
            const FusedLayer &ly = a.layers[l];
            // ---- A: QKV (pair-permuted rows) + RoPE + KV append.
            if (l == 0) stage<true>(xs, emb, H, ly.ln1, a.eps, sm);
            else stage<false>(xs, a.hidden, H, ly.ln1, a.eps, sm);
            const int pairs = (qd + 2 * kvd) / 2;
            for (int j = gw; j < pairs; j += W) {
                const int r0 = 2 * j;
                const uint8_t *rp[2] = {ly.qkv + (size_t)r0 * a.qkv_stride, ly.qkv + (size_t)(r0 + 1) * a.qkv_stride};
                float y[2];
                wave_dots<FMT, UB, 2>(rp, xs, H, y);
                if (lane == 0) {
                    float v0 = y[0], v1 = y[1];
                    if (ly.qkv_sc) {
                        v0 = v0 * ly.qkv_sc[r0];
                        v1 = v1 * ly.qkv_sc[r0 + 1];
                    }
                    v0 = v0 + ly.qkv_bias[r0];
                    v1 = v1 + ly.qkv_bias[r0 + 1];
                    if (r0 < qd + kvd) {
                        const bool is_q = r0 < qd;
                        const int base = is_q ? r0 : r0 - qd;
                        const int h = base / HD, d0 = base % HD;
                        int o0 = d0, o1 = d0 + 1;
                        if (d0 < a.rotary) {
                            const int i = d0 / 2;
                            const float c = cr[i], s = sr[i];
                            const float x1 = v0 * c - v1 * s, x2 = v1 * c + v0 * s;
                            v0 = x1;
                            v1 = x2;
                            o0 = i;
                            o1 = half + i;
                        }
                        if (is_q) {
                            st1(a.qrot + h * HD + o0, v0);
                            st1(a.qrot + h * HD + o1, v1);
                        } else {
                            KT *kc = (KT *)ly.kc + (((size_t)page * a.kv_heads + h) * a.page_size + slot) * HD;
                            st_kv(kc + o0, v0);
                            st_kv(kc + o1, v1);
                        }
                    } else {
                        const int base = r0 - qd - kvd;
                        const int h = base / HD, d0 = base % HD;
                        KT *vc = (KT *)ly.vc + (((size_t)page * a.kv_heads + h) * a.page_size + slot) * HD;
                        st_kv(vc + d0, v0);
                        st_kv(vc + d0 + 1, v1);
                    }
                }
            }
            if (!grid_sync(a, ++epoch, sm)) return;
            // ---- B: attention.
            const int items = a.kv_heads * S;
            for (int it = blockIdx.x; it < items; it += NB) attn_item<HD, G, KT>(a, ly, it / S, it % S, S, ctx, ash);
            if (!grid_sync(a, ++epoch, sm)) return;
            // ---- C: o_proj + residual.
            stage<false>(xs, a.attn, qd, nullptr, 0.f, sm);
            for (int r = gw; r < H; r += W) {
                const uint8_t *rp[1] = {ly.o + (size_t)r * a.o_stride};
                float y[1];
                wave_dots<FMT, UB, 1>(rp, xs, qd, y);
                if (lane == 0) {
                    float v = y[0];
                    if (ly.o_sc) v = v * ly.o_sc[r];
                    if (ly.o_bias) v = v + ly.o_bias[r];
                    const float old = l == 0 ? bf16_f32(emb[r]) : ld1(a.hidden + r);
                    st1(a.hidden + r, old + v);
                }
            }
            if (!grid_sync(a, ++epoch, sm)) return;
            // ---- D: gate/up + SwiGLU.
            stage<false>(xs, a.hidden, H, ly.ln2, a.eps, sm);
            for (int r = gw; r < a.I; r += W) {
                const uint8_t *rp[2] = {ly.gate + (size_t)r * a.gu_stride, ly.up + (size_t)r * a.gu_stride};
                float y[2];
                wave_dots<FMT, UB, 2>(rp, xs, H, y);
                if (lane == 0) {
                    float g = y[0], u = y[1];
                    if (ly.gate_sc) {
                        g = g * ly.gate_sc[r];
                        u = u * ly.up_sc[r];
                    }
                    st1(a.act + r, g * (u / (1.0f + expf(-g))));
                }
            }
            if (!grid_sync(a, ++epoch, sm)) return;
            // ---- E: down + residual.
            stage<false>(xs, a.act, a.I, nullptr, 0.f, sm);
            for (int r = gw; r < H; r += W) {
                const uint8_t *rp[1] = {ly.down + (size_t)r * a.down_stride};
                float y[1];
                wave_dots<FMT, UB, 1>(rp, xs, a.I, y);
                if (lane == 0) {
                    float v = y[0];
                    if (ly.down_sc) v = v * ly.down_sc[r];
                    st1(a.hidden + r, ld1(a.hidden + r) + v);
                }
            }
            if (!grid_sync(a, ++epoch, sm)) return;
        }
        // ---- LM head (BF16, final norm fused) + argmax partials.
        stage<false>(xs, a.hidden, H, a.final_norm, a.eps, sm);
        int key = INT_MIN;
        uint32_t idx = 0;
        const size_t head_stride = (size_t)H * 2;
        for (int r = gw; r < a.V; r += W) {
            const uint8_t *rp[1] = {(const uint8_t *)a.head + (size_t)r * head_stride};
            float y[1];
            wave_dots<FMT_BF16, 16, 1>(rp, xs, H, y);
            if (lane == 0) {
                a.logits[r] = y[0];
                better(key, idx, total_key(y[0]), (uint32_t)r);
            }
        }
        if (lane == 0) {
            stu((unsigned *)a.am_key + gw, (unsigned)key);
            stu(a.am_idx + gw, idx);
        }
        if (!grid_sync(a, ++epoch, sm)) return;
        // Every block reduces the W partials itself.
        key = INT_MIN;
        idx = 0;
        for (int w = tid; w < W; w += kThreads) better(key, idx, (int)ldu((const unsigned *)a.am_key + w), ldu(a.am_idx + w));
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
        token = (int)idx;
        if (blockIdx.x == 0 && tid == 0) {
            if (pos + 1 < a.hist_cap) stu(a.hist + pos + 1, idx);
            stu((unsigned *)a.step, idx);
            stu((unsigned *)a.step + 1, (unsigned)(pos + 1));
        }
        __syncthreads();
    }
    if (blockIdx.x == 0 && tid == 0) stu(a.epoch_base, epoch);
}

template <int FMT, int UB, int HD, int G>
int launch_kt(const FusedArgs &a, int nb, size_t lds, bool kv_f32, hipStream_t s) {
    void *args[] = {(void *)&a};
    if (kv_f32) {
        auto k = decode_fused_kernel<FMT, UB, HD, G, float>;
        CHIP_CHECK(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        CHIP_CHECK(hipLaunchCooperativeKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s));
    } else {
        auto k = decode_fused_kernel<FMT, UB, HD, G, uint16_t>;
        CHIP_CHECK(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        CHIP_CHECK(hipLaunchCooperativeKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s));
    }
    return 0;
}

template <int FMT, int UB>
int launch_fmt(const FusedArgs &a, int nb, size_t lds, int hd, int g, bool kv_f32, hipStream_t s) {
    if (hd == 64 && g == 2) return launch_kt<FMT, UB, 64, 2>(a, nb, lds, kv_f32, s);
    if (hd == 64 && g == 7) return launch_kt<FMT, UB, 64, 7>(a, nb, lds, kv_f32, s);
    if (hd == 128 && g == 4) return launch_kt<FMT, UB, 128, 4>(a, nb, lds, kv_f32, s);
    if (hd == 128 && g == 7) return launch_kt<FMT, UB, 128, 7>(a, nb, lds, kv_f32, s);
    return fail("HIP backend: no persistent decode kernel for this head shape.");
}

}  // namespace

bool fused_decode_supported(int fmt, int head_dim, int group, bool aligned16) {
    if (!((head_dim == 64 && (group == 2 || group == 7)) || (head_dim == 128 && (group == 4 || group == 7))))
        return false;
    if (fmt == FMT_Q4) return true;  // dword units
    return aligned16;
}

int fused_decode_blocks() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

int launch_decode_fused(const FusedArgs &a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s) {
    const int nb = fused_decode_blocks();
    if (nb <= 0) return fail("HIP backend: cannot size the persistent decode grid.");
    const size_t lds = (size_t)std::max(std::max(a.H, a.q_heads * head_dim), a.I) * sizeof(float);
    if (lds + 32768 > device_max_lds()) return fail("HIP backend: persistent decode needs more LDS than a block has.");
    if (fmt == FMT_BF16) return launch_fmt<FMT_BF16, 16>(a, nb, lds, head_dim, group, kv_f32, s);
    if (fmt == FMT_Q8) return launch_fmt<FMT_Q8, 16>(a, nb, lds, head_dim, group, kv_f32, s);
    if (fmt == FMT_Q4) return launch_fmt<FMT_Q4, 4>(a, nb, lds, head_dim, group, kv_f32, s);
    return fail("HIP backend: unknown weight format.");
}

}  // namespace chip
