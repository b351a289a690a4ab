// Persistent dataflow decode kernel interface (decode_fused.hip).
#pragma once

#include "kernels.hpp"

namespace chip {

// One layer's weights as the persistent kernel reads them (device pointers;
// q/k/v pair-permuted, see qkv_perm_row). Scale pointers are null for BF16.
struct FusedLayer {
    const uint8_t *qkv, *o, *gate, *up, *down;
    const float *qkv_sc, *o_sc, *gate_sc, *up_sc, *down_sc;
    const float *qkv_bias;  // f32, pair-permuted like the rows
    const float *o_bias;    // f32 or null
    const uint16_t *ln1, *ln2;
    void *kc, *vc;
    // down_proj columns of each block's gate/up rows, transposed and
    // zero-padded: [blocks][H][rp] BF16 (fused_down_columns).
    const uint16_t *down_cols;
};

// Cross-block values travel as 64-bit words: low half the f32 bits, high
// half the tag of the phase instance that wrote them (never 0, so zeroed
// memory never matches). Every tagged array is followed by at least 2 more
// words of the same allocation, so a 16-byte read at its last word stays in
// bounds.
struct FusedArgs {
    const FusedLayer *layers;  // device array [L]
    int L, H, q_heads, kv_heads, rotary, I, V;
    float eps;
    size_t qkv_stride, o_stride, gu_stride, down_stride;  // payload row strides (bytes)
    const uint16_t *embed, *head, *final_norm;
    const float *rope_cos, *rope_sin;
    const int32_t *page_table;  // 64-position pages
    int32_t *step;              // [0] = token, [1] = position; advanced by the kernel
    uint32_t *hist;
    long hist_cap;
    float *logits;              // [V], the last step's
    uint64_t *hid0, *hid1;      // [H] residual stream after o_proj / after down
    uint64_t *qkvn;             // [kv_heads][(G + 2) * hd]: a group's rotated q heads, then its new K and V rows
    uint64_t *part;             // [max_splits][q_heads][hd + 2] attention partials (output, max, sum)
    uint64_t *pdown;            // [nhb][nbd][7]: gate/up block j's down partial of output rows 7 i .. 7 i + 6
    uint64_t *am;               // [2][blocks][2] argmax partials (key, index) by step parity
    int *abort_flag;            // raised when a poll times out
    unsigned tag0;              // tag of step 0, phase 0 of this launch
    int steps;
    int max_splits;
    long ctx_end;               // context length after the launch's last step
    uint64_t *trace;            // null, or [blocks][16L + 3] phase-end timestamps
    int trace_step;             // the step traced
    // Filled in by launch_decode_fused: dynamic LDS layout (byte offsets) and
    // block roles (o/down blocks, first QKV block, QKV blocks, gate/up rows
    // per block, blocks owning LM-head rows).
    int lds_xs, lds_kv, lds_mw, lds_emb, lds_gain, lds_total;
    int nhb, a0, nab, rb, head_blocks;
    int rp;   // rb rounded up to a multiple of 8 (a down_cols row)
    int nbd;  // blocks that own gate/up rows
};

// Phases per decode step: 5 per layer (qkv, attention, o, gate/up, down) + head.
__host__ __device__ constexpr int fused_phases_per_step(int layers) { return 5 * layers + 1; }

// Positions one attention work item covers (one block; K and V in LDS).
int fused_positions_per_item(int head_dim, bool kv_f32);

// Whether a kernel is built for this model shape on `blocks` blocks.
bool fused_decode_supported(int fmt, int H, int q_heads, int kv_heads, int head_dim, int I, bool aligned16,
                            int blocks);
int fused_decode_blocks();

// Largest attention split count the kernel's LDS holds for this shape
// (capped by the grid and by `capacity` positions); 0 if none fits.
int fused_max_splits(int H, int q_heads, int kv_heads, int head_dim, int I, bool kv_f32, int blocks,
                     size_t capacity);

// Gate/up rows per block and their padded count on `blocks` blocks.
inline int fused_gate_rows(int I, int blocks) { return (I + blocks - 1) / blocks; }
inline int fused_gate_rows_padded(int I, int blocks) { return (fused_gate_rows(I, blocks) + 7) / 8 * 8; }

// Writes dst[b][r][j] = down[r][b * rb + j] (BF16; 0 for j >= rb or a
// column past I), rb = fused_gate_rows(I, blocks), for b < blocks, r < H,
// j < fused_gate_rows_padded(I, blocks). down rows are `stride` bytes apart.
int fused_down_columns(const uint16_t *down, size_t stride, int H, int I, int blocks, uint16_t *dst, hipStream_t s);

// Fills in a.lds_* and launches (a is taken by value for that).
int launch_decode_fused(FusedArgs a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s);

}  // namespace chip
