/*
 * cheetah_ref_cpu — CPU oracle for the decoder forward.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in C++, the arithmetic of
 * Cheetah's native CPU backend (Rust, not buildable here: no rustc/cargo).
 * It is the checker for the HIP library's parity tests and the CPU baseline
 * timed next to the GPU numbers. Nothing in the product path may link, load
 * or call it.
 *
 * Every function cites the reference file:line whose arithmetic it follows.
 * Build: -O3 -mavx2 -mfma -ffp-contract=off. FMA appears only where the
 * reference uses explicit FMA intrinsics (the BF16 dot kernels); everything
 * else is separately rounded, in the reference's left-to-right order.
 */
#ifndef CHEETAH_REF_CPU_H
#define CHEETAH_REF_CPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- math kernels (src/chat/native/ops.rs) ---- */
void ref_set_threads(int threads);
int ref_get_threads(void);

/* dtype codes: 0 = F32, 1 = BF16 (WeightDType, src/chat/native/store.rs:13-39) */
void ref_gemv(const void *weight, int dtype, size_t rows, size_t cols,
              const float *x, float *y);
void ref_gemm_bf16(const uint16_t *weight, size_t rows, size_t cols,
                   const float *x, size_t n, float *y);
void ref_gemv_q8(const uint8_t *buffer, size_t rows, size_t cols,
                 const float *x, float *y);
void ref_gemv_q4(const uint8_t *buffer, size_t rows, size_t cols,
                 const float *x, float *y);
/* n tokens through gemv_q8 (fmt 4) / gemv_q4 (fmt 5) at once; bit-identical
 * to n per-token calls (the reference's linear_batch for quantized units,
 * ops.rs:1244-1326). y is [n][rows]. */
void ref_gemm_quant(const uint8_t *buffer, uint32_t fmt, size_t rows, size_t cols,
                    const float *x, size_t n, float *y);
size_t ref_q8_buffer_bytes(size_t rows, size_t cols);
size_t ref_q4_buffer_bytes(size_t rows, size_t cols);
size_t ref_q4_row_stride(size_t cols);
int ref_quantize_q8(const float *values, size_t rows, size_t cols,
                    uint8_t *out, size_t out_len);
int ref_quantize_q4(const float *values, size_t rows, size_t cols,
                    uint8_t *out, size_t out_len);
float ref_q8_dequant_value(const uint8_t *buffer, size_t rows, size_t cols,
                           size_t row, size_t col);
float ref_q4_dequant_value(const uint8_t *buffer, size_t rows, size_t cols,
                           size_t row, size_t col);
void ref_rmsnorm(float *x, size_t n, const uint16_t *weight_bf16, float eps);
void ref_rope_in_place(float *values, size_t heads, size_t head_dim,
                       size_t position, float theta);
void ref_rope_heads(float *values, size_t heads, size_t head_dim,
                    size_t rotary_dim, size_t position, float theta);
void ref_silu_multiply(float *gate, const float *up, size_t n);
/* The BF16-KV mode's rounding of each appended K/V element (f32 -> BF16,
 * nearest, ties to even), as values widened back to f32. */
void ref_round_bf16(const float *in, float *out, size_t n);
void ref_softmax(float *scores, size_t n);
/* GQA attention of one query position over a contiguous f32 cache laid out
 * [pos][kv_head][head_dim] (ops.rs:1357-1467). */
void ref_attention(const float *keys, const float *values, size_t cache_len,
                   const float *q, float *out, size_t q_heads, size_t kv_heads,
                   size_t head_dim, size_t position, size_t sliding_window);
/* `rows` query rows of one chunk at positions offset..offset+rows-1 over a
 * cache already holding offset+rows positions; row r sees the first
 * offset+r+1. Bit-identical to ref_attention per row (ops.rs:1357-1467). */
void ref_attention_rows(const float *keys, const float *values, size_t offset,
                        size_t rows, const float *q, float *out, size_t q_heads,
                        size_t kv_heads, size_t head_dim, size_t sliding_window);

/* ---- model (src/chat/registrations/{qwen2,llama}.rs) ---- */
typedef struct ref_config {
    uint32_t num_layers;
    uint32_t hidden_size;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;
    uint32_t intermediate_size;
    uint32_t vocab_size;
    uint32_t tie_word_embeddings;
    uint32_t sliding_window;
    float rope_theta;
    float rms_eps;
} ref_config;

typedef struct ref_model ref_model;
typedef struct ref_snapshot ref_snapshot;

/* quant_format: 0 = stored precision, 4 = q8, 5 = q4 (precision.rs registry
 * order: CHEETAH_QUANT_Q8 / CHEETAH_QUANT_Q4). kv_bf16 != 0 rounds appended
 * K/V rows to BF16 (round-to-nearest-even) to model a BF16 KV cache; the
 * reference keeps f32 (kv_bf16 = 0). */
ref_model *ref_model_create(const ref_config *cfg, uint32_t quant_format,
                            int kv_bf16);
/* Registers one weight unit (borrowed bytes, like the mmap store slice,
 * store.rs:189-203). dtype as above. */
int ref_model_set_unit(ref_model *m, const char *unit_id, const void *bytes,
                       size_t nbytes, int dtype, const uint64_t *shape,
                       size_t ndim);
int ref_model_forward(ref_model *m, const uint32_t *tokens, size_t n,
                      size_t offset, size_t chunk_rows, float *logits);
void ref_model_clear_cache(ref_model *m);
ref_model *ref_model_clone(const ref_model *m);
size_t ref_model_kv_len(const ref_model *m);
ref_snapshot *ref_model_kv_snapshot(const ref_model *m);
int ref_model_restore_kv_prefix(ref_model *m, const ref_snapshot *s,
                                size_t positions);
size_t ref_snapshot_positions(const ref_snapshot *s);
void ref_snapshot_free(ref_snapshot *s);
void ref_model_free(ref_model *m);
const char *ref_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
