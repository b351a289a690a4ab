// Persistent decode kernel interface (decode_fused.hip).
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
};

struct FusedArgs {
    const FusedLayer *layers;  // device array [L]
    int L, H, q_heads, kv_heads, rotary, I, V;
    float eps;
    size_t qkv_stride, o_stride, gu_stride, down_stride;  // payload row strides (bytes)
    const uint16_t *embed, *head, *final_norm;
    const float *rope_cos, *rope_sin;
    const int32_t *page_table;
    int page_size;
    int32_t *step;  // [0] = token, [1] = position; advanced by the kernel
    uint32_t *hist;
    long hist_cap;
    float *hidden, *qrot, *part, *attn, *act, *logits;
    int *am_key;
    uint32_t *am_idx;       // [blocks * 4] argmax partials
    unsigned *arrive;       // [blocks] barrier arrival epochs
    unsigned *go;           // barrier release epoch
    unsigned *epoch_base;   // last epoch of the previous launch
    unsigned *attn_count;   // [kv_heads] split arrival counters, zero at rest
    int *abort_flag;        // raised when a barrier spin times out
    int steps;
    int max_splits;         // at most 64
};

bool fused_decode_supported(int fmt, int head_dim, int group, bool aligned16);
int fused_decode_blocks();
int launch_decode_fused(const FusedArgs &a, int fmt, int head_dim, int group, bool kv_f32, hipStream_t s);

}  // namespace chip
