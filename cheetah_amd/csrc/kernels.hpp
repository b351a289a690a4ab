// Host-side launchers of the gfx950 kernels. Every launcher validates the
// shapes it is given before touching the device and returns 0 / -1.
#pragma once

#include "common.hpp"

namespace chip {

// Largest LDS allocation one block may make (queried at init).
size_t device_max_lds();
int device_cus();
size_t device_lds_per_cu();

// ---------------------------------------------------------------------------
// Weight matrix in device memory, in the reference's layout.
// ---------------------------------------------------------------------------
struct WMat {
    int fmt = FMT_BF16;
    const uint8_t *base = nullptr;  // start of the buffer (scale head first for q8/q4)
    size_t rows = 0, cols = 0;
    const float *scales() const { return fmt == FMT_BF16 ? nullptr : (const float *)base; }
    const uint8_t *payload() const { return fmt == FMT_BF16 ? base : base + rows * 4; }
    size_t row_stride() const { return fmt_row_bytes(fmt, cols); }
    size_t bytes() const { return fmt_buffer_bytes(fmt, rows, cols); }
};

// Epilogue of a GEMV / GEMM: out = f(acc * row_scale (+ bias)).
enum Epi : int {
    EPI_STORE = 0,     // y = v
    EPI_RESIDUAL = 1,  // residual += v            (y unused)
    EPI_SWIGLU = 2,    // y = g * (u / (1 + exp(-g)))  (dual matrix: gate, up)
};

struct GemvJob {
    WMat w;              // the matrix (gate for EPI_SWIGLU)
    WMat w2;             // up matrix for EPI_SWIGLU
    const float *x = nullptr;        // input vector [cols] (hidden when norm_gain is set)
    const uint16_t *norm_gain = nullptr;  // BF16 RMSNorm gain: x := rmsnorm(x) first
    float eps = 0.f;
    const float *bias = nullptr;     // f32 [rows]
    float *y = nullptr;              // output [rows]
    float *residual = nullptr;       // EPI_RESIDUAL target [rows]
    int epi = EPI_STORE;
};
int launch_gemv(const GemvJob &job, hipStream_t stream);

struct GemmJob {
    WMat w, w2;
    const float *x = nullptr;  // [n][cols] f32
    size_t n = 0;
    const float *bias = nullptr;
    float *y = nullptr;          // [n][rows]
    float *residual = nullptr;   // [n][rows]
    int epi = EPI_STORE;
    // Optional split-K scratch; without room for the chunk sums the GEMM
    // folds in registers (the same bits, fewer blocks).
    float *ws = nullptr;
    size_t ws_floats = 0;
    // Optional x pre-split by launch_split_bf16 ([n][cols] each): the GEMM
    // then stages BF16 halves instead of splitting x once per weight tile
    // (the same bits).
    const uint16_t *xh = nullptr, *xl = nullptr;
    // EPI_SWIGLU only, optional: the output also as BF16 halves ([n][rows]
    // each, the bits launch_split_bf16 would give), for the next GEMM.
    uint16_t *yh = nullptr, *yl = nullptr;
    // EPI_RESIDUAL / EPI_STORE, optional: when the GEMM splits K, leave the
    // stored sums in ws ([*deferred][n][rows]: every chunk's, or the two
    // halves') for the caller's reduction (launch_residual_rmsnorm_rows,
    // launch_rope_append) and set *deferred to their count; 0 when the GEMM
    // applied its epilogue itself.
    int *deferred = nullptr;
};
int launch_gemm(const GemmJob &job, hipStream_t stream);
int launch_split_bf16(const float *x, size_t n, uint16_t *xh, uint16_t *xl, hipStream_t s);
int gemm_chunk_depth(int K);
size_t gemm_workspace_floats(size_t N, size_t K, size_t M, bool dual);
// Scratch the split path can use for any token count up to m_max.
size_t gemm_split_workspace_floats(size_t N, size_t K, size_t m_max, bool dual);

// ---------------------------------------------------------------------------
// Quantization (bit-exact to q8.rs / q4.rs quantize) and dequantization.
// ---------------------------------------------------------------------------
int launch_quantize(int fmt, const uint16_t *w_bf16, size_t rows, size_t cols, uint8_t *out, hipStream_t s);
int launch_dequant(const WMat &w, float *out, hipStream_t s);

// ---------------------------------------------------------------------------
// Small ops.
// ---------------------------------------------------------------------------
// hidden[i][:] = bf16 table[tokens[i]][:]
int launch_embed(const uint16_t *table, size_t hidden, const uint32_t *tokens, size_t rows, float *out,
                 hipStream_t s);
// out[i][:] = rmsnorm(x[i][:]) * gain (rows of width n)
// Row-wise RMSNorm; with xh / xl also the normed rows as BF16 halves (the
// bits launch_split_bf16 would give), the MFMA GEMM's input.
int launch_rmsnorm_rows(const float *x, const uint16_t *gain, float eps, size_t rows, size_t n, float *out,
                        hipStream_t s, uint16_t *xh = nullptr, uint16_t *xl = nullptr);
// A deferred residual GEMM's reduction fused with the next RMSNorm: per row
// m and column i, v = the nchunks stored sums ws[z][m][i] folded as the
// GEMM folds them (the first ceil(n / 2) in order, the rest in order, the
// two added), times
// sc[i], plus bias[i] (each optional), hidden[m][i] += v; then, with a gain,
// the row RMSNorm of hidden into out (and BF16 halves when xh / xl are set).
// The same operations as the GEMM's split-K reduction then
// launch_rmsnorm_rows.
int launch_residual_rmsnorm_rows(const float *ws, int nchunks, const float *sc, const float *bias, float *hidden,
                                 size_t rows, size_t n, const uint16_t *gain, float eps, float *out, hipStream_t s,
                                 uint16_t *xh = nullptr, uint16_t *xl = nullptr);

// Paged KV cache of one layer: [pages][kv_heads][page_size][head_dim]
// elements, BF16 (default) or f32 (the reference's own cache precision).
struct KvLayer {
    void *k = nullptr;
    void *v = nullptr;
};
struct KvGeom {
    const int32_t *page_table = nullptr;  // device
    int page_size = 64;
    int kv_heads = 0;
    int head_dim = 0;
    int kv_f32 = 0;  // 0 = BF16 elements, 1 = f32 elements
};

// The q/k rows of a layer's packed QKV matrix are stored pair-permuted: in
// every head, output rows i and i + rotary_dim/2 (the two halves a RoPE
// rotation mixes) sit next to each other at 2i and 2i + 1; dims at or past
// rotary_dim keep their place; v rows are unpermuted. qkv_perm_row maps a
// stored row to the reference row it holds.
int qkv_perm_row(int stored_row, int q_heads, int kv_heads, int head_dim, int rotary_dim);

// RoPE (rotate-half, host cos/sin table) on the q and k parts of packed,
// pair-permuted qkv rows [rows][q_dim + 2*kv_dim]: rotated q goes to
// qrot[rows][q_dim] in reference order, K and V rows are appended to the
// paged cache. Positions are pos0 + i, where pos0 is read from *pos_dev when
// pos_dev is set (decode graph) and is `offset` otherwise.
// With nchunks > 0 the qkv values are a deferred split-K GEMM's: the stored
// sums ws[nchunks][rows][q_dim + 2*kv_dim] folded as the GEMM folds them (the
// first ceil(n / 2) in order, the rest in order, the two added), times sc (if
// set), plus bias (if set) - the GEMM epilogue's arithmetic; qkv is unused.
int launch_rope_append(const float *qkv, float *qrot, size_t rows, int q_heads, const KvGeom &g, const KvLayer &kv,
                       const float *rope_cos, const float *rope_sin, int rotary_dim, size_t offset,
                       const int32_t *pos_dev, hipStream_t s, const float *ws = nullptr, int nchunks = 0,
                       const float *sc = nullptr, const float *bias = nullptr);

// dst[r][:] = src[map[r]][:] for rows of row_bytes bytes (load-time layout).
int launch_gather_rows(const uint8_t *src, uint8_t *dst, const int32_t *map, size_t rows, size_t row_bytes,
                       hipStream_t s);

// GQA attention for `rows` query rows at positions pos0 + i over keys
// [0, pos0 + i]. q row stride q_stride floats. The split count (at most
// attention_max_splits()) is the caller's: decode graphs need a fixed grid.
// Partial buffers hold rows * q_heads * splits * (head_dim + 2) floats.
// Keys per split of the matrix-core chunked prefill when the caller names
// no span (attention_prefill_span gives a model's).
constexpr int kDefaultPrefillSpan = 1024;

struct AttnJob {
    const float *q = nullptr;
    size_t q_stride = 0;
    float *out = nullptr;  // [rows][q_heads*head_dim]
    const void *k = nullptr, *v = nullptr;
    KvGeom g;
    int q_heads = 0;
    size_t rows = 0;
    size_t offset = 0;
    const int32_t *pos_dev = nullptr;
    int splits = 1;
    float *part = nullptr;  // partial buffer (splits > 1)
    // Chunked prefill (host offset): BF16 KV with head_dim 64/128 runs on the
    // matrix cores with attention_prefill_splits(offset + rows) splits and
    // ignores `splits`; part must then hold part_floats >= the partials.
    bool prefill = false;
    size_t part_floats = 0;
    // Keys per prefill split (absolute position ranges [s span, (s+1) span)):
    // a row's bits depend on it, so a model keeps one span for its lifetime.
    int span = kDefaultPrefillSpan;
    // Decode (one row) from the raw QKV row [q | k | v] of launch_rope_append
    // instead of q: the kernel rotates q itself and rotates and appends the
    // position's K/V row (what launch_rope_append would write; q unused).
    // Only where attention_decode_fuses_rope says so.
    const float *qkv = nullptr;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    int rotary_dim = 0;
    // Chunked prefill on the matrix cores (attention_prefill_on_mfma) also
    // writes out's BF16 halves here when set: hi = bf16(v), lo = bf16(v - hi),
    // the bits launch_split_bf16 would write. Other paths ignore them.
    uint16_t *out_hi = nullptr, *out_lo = nullptr;
};
int launch_attention(const AttnJob &job, hipStream_t s);
// BF16 K/V on the matrix cores, head_dim 64/128, <= 8 q heads per KV head,
// rotary width = head_dim.
bool attention_decode_fuses_rope(const KvGeom &g, int q_heads, int rotary_dim);
size_t attention_part_floats(size_t rows, int q_heads, int splits, int head_dim);
// Split count of a decode-style launch (one row per query position) over ctx
// keys: one or two blocks per CU (matrix-core or VALU kernel), at most one
// split per 64-position tile.
int attention_decode_splits(size_t ctx, int kv_heads, size_t rows, bool kv_f32);
int attention_max_splits();
int attention_prefill_splits(size_t ctx, int span = kDefaultPrefillSpan);
// A model's prefill span from its KV capacity: the largest power of two at
// most capacity / 8, and at least kDefaultPrefillSpan.
int attention_prefill_span(size_t kv_capacity);
bool attention_prefill_on_mfma(const KvGeom &g, int q_heads);

// Greedy argmax (ties -> last index, total order) of logits[n]; writes the
// index to *out_token. When `step` is set (the device-side decode loop,
// step[0] = token, step[1] = position) it also records the index as the
// token of position step[1] + 1 in hist[] (when that is < hist_cap), stores
// it in step[0] and advances step[1] by one.
int launch_argmax(const float *logits, size_t n, uint32_t *out_token, int32_t *step, uint32_t *hist,
                  size_t hist_cap, void *scratch, hipStream_t s);
size_t argmax_scratch_bytes();

}  // namespace chip
