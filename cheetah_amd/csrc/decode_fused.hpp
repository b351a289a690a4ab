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
    // down_proj columns of each FFN block's gate/up rows, transposed and
    // zero-padded: [ffn blocks][H][rp] BF16 (fused_down_columns).
    const uint16_t *down_cols;
};

// How the grid divides into roles for one model shape (fused_geometry).
//   items:  one q head over one run of `ip` positions each: item (split s,
//           head h) at block s * qp + slot(h), qp = q_heads rounded up to 8
//           (the XCD count), slot(h) from fused_item_slots, item index
//           s * q_heads + h
//   KV:     blocks [kv0, kv0 + nkv): the new position's K/V rows, one
//           rotation pair per wave
//   FFN:    blocks [f0, f0 + nf): gate/up rows, SwiGLU, down columns; the
//           first `no` of them also own 8 residual rows each
struct FusedGeom {
    int nf, f0;        // FFN blocks
    int nkv, kv0;      // KV blocks
    int s_cap;         // attention splits per q head the item blocks hold
    int ip_max;        // longest run of positions one item holds in LDS
    int no;            // residual owner blocks (8 rows each)
    int rb, rp, nbd;   // gate/up rows per FFN block, padded to 8, FFN blocks with rows
    int ni_max;        // q_heads * s_cap
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
    uint64_t *hid0, *hid1;      // [H] residual stream after attention / after the MLP
    uint64_t *kvw;              // [kv_heads][2 hd]: the new position's rotated K row, then its V row
    uint64_t *part;             // [no][ni][8]: item i's o_proj partial of owner o's 8 rows
    uint64_t *ml;               // [ni][2]: item i's max score and sum of weights
    uint64_t *pdown;            // [no][nbd][8]: FFN block f's down partial of owner o's 8 rows
    uint64_t *am;               // [2][blocks][2] argmax partials (key, index) by step parity
    int *abort_flag;            // raised when a poll times out
    unsigned tag0;              // tag of step 0, phase 0 of this launch
    int steps;
    long ctx_end;               // context length after the launch's last step
    uint64_t *trace;            // null, or [blocks][16L + 3] phase-end timestamps
    int trace_step;             // the step traced
    // Filled in by launch_decode_fused: roles (FusedGeom), the launch's
    // split count and positions per item, and the dynamic LDS layout (byte
    // offsets).
    int ni, ip, splits;         // items (q_heads * splits), positions per item
    int kv0, nkv, f0, nf, no, nbd, rb, rp, head_blocks;
    // Item placement: the q head of each of the heads_padded block slots of
    // a run (slot j on XCD j % 8), or -1 for a slot without an item.
    int32_t slot_head[64];  // 32-bit: read by scalar loads (a byte would take a vector load)
    int lds_xs, lds_xb, lds_q, lds_kv, lds_emb, lds_g1, lds_g2, lds_total;
};

// Phases per decode step: 5 per layer (new K/V, item partials, attention
// residual, down partials, MLP residual) + the LM head.
__host__ __device__ constexpr int fused_phases_per_step(int layers) { return 5 * layers + 1; }

// Whether a kernel is built for this model shape on `blocks` blocks, and
// the role geometry it uses (valid when supported).
bool fused_decode_supported(int fmt, int H, int q_heads, int kv_heads, int head_dim, int I, bool aligned16,
                            int blocks);
FusedGeom fused_geometry(int H, int q_heads, int kv_heads, int head_dim, int I, bool kv_f32, int blocks);
int fused_decode_blocks();

// Longest context one launch can reach: s_cap splits of ip_max positions.
inline long fused_max_context(const FusedGeom &g) { return (long)g.s_cap * g.ip_max; }

// Gate/up rows per FFN block and their padded count on `nf` FFN blocks.
inline int fused_gate_rows(int I, int nf) { return (I + nf - 1) / nf; }
inline int fused_gate_rows_padded(int I, int nf) { return (fused_gate_rows(I, nf) + 7) / 8 * 8; }

// Writes dst[b][r][j] = down[r][b * rb + j] (BF16; 0 for j >= rb or a
// column past I), rb = fused_gate_rows(I, nf), for b < nf, r < H,
// j < fused_gate_rows_padded(I, nf). down rows are `stride` bytes apart.
int fused_down_columns(const uint16_t *down, size_t stride, int H, int I, int nf, uint16_t *dst, hipStream_t s);

// Fills in the roles, the launch's splits and the LDS layout (a is taken by
// value for that) and launches.
int launch_decode_fused(FusedArgs a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s);

}  // namespace chip
