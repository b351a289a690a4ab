/*
 * cheetah_hip.h — C-ABI of the MI355X (gfx950) decoder-forward backend for
 * Cheetah's `ModelForward` boundary (CHEETAH_DEVICE=hip).
 *
 * Conventions follow the reference's device C-ABI (cheetah_vulkan.h):
 *  - int status: 0 on success, -1 on failure; the failure sentence is kept
 *    per thread and read with cheetah_hip_last_error() (the Rust wrapper maps
 *    it to Err(String), as src/native.rs:1860-1870 does for Vulkan);
 *  - caller-owned output buffers, plain pointers and sizes, opaque handles;
 *  - every argument error is rejected before any device work.
 *
 * Pointers documented as "device" point to memory from cheetah_hip_alloc();
 * everything else is host memory.
 */
#ifndef CHEETAH_HIP_H
#define CHEETAH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * Lifecycle. Replaces init_vulkan_device / shutdown_vulkan_device
 * (cheetah_vulkan.h:15-16). Fails on anything but a gfx950 device.
 * ---------------------------------------------------------------------- */
int cheetah_hip_init(int device);
void cheetah_hip_shutdown(void);
/* Backend label for the banner (registry.rs:62 ModelForward::device_name). */
const char *cheetah_hip_device_name(void);
const char *cheetah_hip_last_error(void);

/* ------------------------------------------------------------------------
 * Device memory. Replaces vk_alloc_vram / vk_free_vram
 * (cheetah_vulkan.h:22-23). All copies are synchronous.
 * ---------------------------------------------------------------------- */
void *cheetah_hip_alloc(size_t bytes);
int cheetah_hip_free(void *device_ptr);
int cheetah_hip_upload(void *device_dst, const void *host_src, size_t bytes);
int cheetah_hip_download(void *host_dst, const void *device_src, size_t bytes);
/* Device-to-device copy. No counterpart in the reference; measurement
 * helper (the plain copy whose byte counters calibrate the HBM traffic of
 * the other kernels). */
int cheetah_hip_copy(void *device_dst, const void *device_src, size_t bytes);
int cheetah_hip_synchronize(void);

/* ------------------------------------------------------------------------
 * Op-level entry points (device pointers; run on the library stream and
 * return after the work is queued — call cheetah_hip_synchronize() or a
 * download before reading results).
 *
 * Weight layouts are the reference's own:
 *  - BF16: row-major [rows][cols] uint16 bits;
 *  - Q8:  rows f32 row scales, then rows payload rows of (cols+3)/4*4 int8
 *         codes (src/chat/precision/q8.rs:1-25);
 *  - Q4:  rows f32 row scales, then rows payload rows of
 *         ceil(ceil((cols+1)/2)/4)*4 bytes, two int4 codes per byte, low
 *         nibble = even column (src/chat/precision/q4.rs:1-52).
 * ---------------------------------------------------------------------- */

/* y[rows] = W[rows, cols] · x[cols]. Replaces gemv (ops.rs:246), gemv_q8
 * (ops.rs:544), gemv_q4 (ops.rs:586) and the resident Vulkan matmuls
 * (vk_matmul_{bf16,q8,q4}_transposed_resident_checked, native.rs:987-1030). */
int cheetah_hip_gemv_bf16(const uint16_t *w, size_t rows, size_t cols, const float *x, float *y);
int cheetah_hip_gemv_q8(const uint8_t *w, size_t rows, size_t cols, const float *x, float *y);
int cheetah_hip_gemv_q4(const uint8_t *w, size_t rows, size_t cols, const float *x, float *y);

/* Y[n, rows] = X[n, cols] · Wᵀ. Replaces gemm (ops.rs:308) and the
 * per-row quantized linear_batch loop (ops.rs:1244-1326). */
int cheetah_hip_gemm_bf16(const uint16_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y);
int cheetah_hip_gemm_q8(const uint8_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y);
int cheetah_hip_gemm_q4(const uint8_t *w, size_t rows, size_t cols, const float *x, size_t n, float *y);

/* Row-wise quantization of a BF16 matrix into the reference layouts,
 * bit-exact to q8::quantize (q8.rs:91-125) / q4::quantize (q4.rs:126-161).
 * out_len must equal the layout's byte length. */
size_t cheetah_hip_q8_buffer_bytes(size_t rows, size_t cols);
size_t cheetah_hip_q4_buffer_bytes(size_t rows, size_t cols);
int cheetah_hip_quantize_q8(const uint16_t *w_bf16, size_t rows, size_t cols, uint8_t *out, size_t out_len);
int cheetah_hip_quantize_q4(const uint16_t *w_bf16, size_t rows, size_t cols, uint8_t *out, size_t out_len);
/* out[rows, cols] = scale[row] * code[row, col] (Q8Matrix/Q4Matrix::
 * dequant_value, q8.rs / q4.rs:101-110): the in-register dequantization
 * the GEMV/GEMM kernels use, written out for bit-exact checks. */
int cheetah_hip_dequant_q8(const uint8_t *w, size_t rows, size_t cols, float *out);
int cheetah_hip_dequant_q4(const uint8_t *w, size_t rows, size_t cols, float *out);

/* Paged BF16 KV cache view. K and V pools are
 * [pages][kv_heads][page_size][head_dim] BF16; page_table maps logical page
 * (position / page_size) to a physical page (device int32). */
typedef struct cheetah_hip_kv_view {
    const uint16_t *k_pages;
    const uint16_t *v_pages;
    const int32_t *page_table;
    uint32_t page_size;
    uint32_t kv_heads;
    uint32_t head_dim;
} cheetah_hip_kv_view;

/* GQA causal attention (ops.rs:1357-1467 attention / attention_head) for
 * `rows` query rows at absolute positions offset .. offset+rows-1; query row
 * i attends to cached positions [0, offset+i] (their K/V already in the
 * cache). q: device f32 [rows][q_heads*head_dim] (post-rope); out: device
 * f32 [rows][q_heads*head_dim]. Decode is rows == 1. */
int cheetah_hip_attention(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                          size_t offset, float *out);
/* cheetah_hip_attention that allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). The split partials live
 * in a fixed 48 MiB device array per GPU instead of a buffer the library
 * grows on demand; a call that needs more (rows * q_heads * splits *
 * (head_dim + 2) floats) is rejected with an error before any device work.
 * Same kernels and split choice, so the same results as
 * cheetah_hip_attention. Like every op-level entry point it launches on the
 * library's own stream (created by cheetah_hip_init; cheetah_hip_synchronize
 * waits for it), not on a stream of the caller's: it is not captured by a
 * graph capture the caller runs on its own stream. Calls within a process
 * are therefore ordered on that one stream and do not overlap on the
 * device; the array keeps the last call's partials. */
int cheetah_hip_attention_noalloc(const float *q, const cheetah_hip_kv_view *kv, uint32_t q_heads, size_t rows,
                                  size_t offset, float *out);

/* ------------------------------------------------------------------------
 * Model: the HIP implementation of ModelForward (registry.rs:57-85) for the
 * qwen2 and llama families (registrations/qwen2.rs, llama.rs).
 * ---------------------------------------------------------------------- */
typedef struct cheetah_hip_config {
    uint32_t family; /* 0 = qwen2, 1 = llama */
    uint32_t num_layers;
    uint32_t hidden_size;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rotary_dim;
    uint32_t intermediate_size;
    uint32_t vocab_size;
    uint32_t tie_word_embeddings;
    uint32_t sliding_window; /* 0 = whole cache (the only value served) */
    float rope_theta;
    float rms_eps;
} cheetah_hip_config;

typedef struct cheetah_hip_model cheetah_hip_model;
typedef struct cheetah_hip_snapshot cheetah_hip_snapshot;

/* Creates a model shell. quant_format: 0 = stored precision (BF16), 4 = q8,
 * 5 = q4 (CHEETAH_QUANT_Q8 / CHEETAH_QUANT_Q4, precision.rs:333-356; linear
 * projections only — embedding, head, norms and biases keep BF16,
 * ops.rs:1533-1537). kv_format: element type of the paged KV cache, 0 = BF16
 * (half the KV bytes), 1 = f32 (the reference's own cache precision,
 * ops.rs:995-999). kv_capacity: positions the KV pool holds across this
 * model, its clones and its snapshots (0 = 65536). max_chunk_rows: largest
 * prefill chunk (0 = 1024). */
cheetah_hip_model *cheetah_hip_model_create(const cheetah_hip_config *cfg, uint32_t quant_format,
                                            uint32_t kv_format, size_t kv_capacity, size_t max_chunk_rows);
/* Uploads one weight unit (host bytes, as MmapWeightStore::slice serves
 * them, store.rs:189-203). dtype: 1 = BF16 (the only stored precision
 * served). Unit ids are the safetensors names ("model.layers.3.mlp.up_proj.weight"). */
int cheetah_hip_model_set_unit(cheetah_hip_model *m, const char *unit_id, const void *bytes, size_t nbytes,
                               uint32_t dtype, const uint64_t *shape, size_t ndim);
/* Checks every unit is present with its shape, builds the fused device
 * layouts and quantizes (the load-time half of ops.rs:1199-1226). */
int cheetah_hip_model_finalize(cheetah_hip_model *m);

/* ModelForward::forward (registry.rs:60): runs tokens[0..n) from absolute
 * position `offset` (must equal the cached length, transformer.rs:799-810)
 * and writes the final position's logits (vocab_size floats) to logits_out.
 * n == 1 runs the decode step; n > 1 runs chunked prefill in chunks of
 * chunk_rows (0 = 256, CHEETAH_PREFILL_CHUNK default, ops.rs:519-535). */
int cheetah_hip_forward(cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset,
                        size_t chunk_rows, float *logits_out);
/* forward + greedy sampling on the device (engine.rs:2247-2253: argmax,
 * ties to the last index). logits_out may be NULL. */
int cheetah_hip_forward_greedy(cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset,
                               size_t chunk_rows, uint32_t *next_token, float *logits_out);
/* The greedy decode loop of Engine::generate_inner (engine.rs:1920-1961)
 * kept on the device: starting from `token` at position `offset`, runs
 * `steps` decode forwards, each feeding its argmax to the next, and writes
 * the sampled ids to tokens_out[steps]. */
int cheetah_hip_decode_greedy(cheetah_hip_model *m, uint32_t token, size_t offset, size_t steps,
                              uint32_t *tokens_out);
/* ModelForward::clear_cache (registry.rs:62). */
void cheetah_hip_clear_cache(cheetah_hip_model *m);
/* Boxed clone per generation (registry.rs:95-117, ops.rs:1017-1029): shares
 * weights and the KV page pool, starts with an empty cache. */
cheetah_hip_model *cheetah_hip_clone(const cheetah_hip_model *m);
size_t cheetah_hip_kv_len(const cheetah_hip_model *m);
/* ModelForward::kv_snapshot / restore_kv_prefix (registry.rs:68-79). A
 * snapshot holds references to the model's KV pages (no copy); a restore
 * maps the first `positions` positions into an empty model and copies a
 * page only when it is next written (copy on write). */
int cheetah_hip_kv_snapshot(const cheetah_hip_model *m, cheetah_hip_snapshot **out, size_t *positions);
int cheetah_hip_restore_kv_prefix(cheetah_hip_model *m, const cheetah_hip_snapshot *s, size_t positions);
void cheetah_hip_snapshot_free(cheetah_hip_snapshot *s);
/* Cached K and V rows of positions [pos_begin, pos_begin + n) of one layer,
 * written to host buffers of n * kv_heads * head_dim floats each in the
 * reference's per-layer cache layout [pos][kv_head][dim] (ops.rs:995-999,
 * the rows KvSnapshot carries, registry.rs:48-55). BF16 pages widen exactly.
 * Waits for the model's queued work. */
int cheetah_hip_kv_download(const cheetah_hip_model *m, uint32_t layer, size_t pos_begin, size_t n, float *k_out,
                            float *v_out);
void cheetah_hip_model_free(cheetah_hip_model *m);

/* Ant tier control (AntTierControl::page_in_unit / evict_unit,
 * registry.rs:87-93; called from engine.rs:1210-1226). The movable units
 * are the per-layer linear weights, model.layers.{l}.self_attn.{q,k,v,o}_proj
 * .weight and model.layers.{l}.mlp.{gate,up,down}_proj.weight; q, k and v
 * name one fused matrix and move together.
 *   evict:   the device buffer is released and a pinned host copy becomes
 *            authoritative (vulkan/transformer.rs:578-583). Forwards keep
 *            working: each such layer's matrices are copied into one of two
 *            device slots on a second stream, one streamed layer ahead of
 *            the compute, with the same kernels reading them there (results
 *            are bit-identical). While any unit is evicted, decode runs the
 *            per-kernel path (no persistent kernel, no captured graph).
 *   page_in: the unit returns to HBM and its host copy is freed; `tier` is
 *            accepted and ignored, as every reference implementation does
 *            (vulkan/transformer.rs:572-576).
 * Both return 1 when the id names a movable unit (also when it already sits
 * in the requested tier), 0 for any other id, -1 on error. They wait for the
 * device to go idle and change weights shared with every clone: they must
 * not overlap a forward on any instance sharing them. */
int cheetah_hip_evict_unit(cheetah_hip_model *m, const char *unit_id);
int cheetah_hip_page_in_unit(cheetah_hip_model *m, const char *unit_id, int32_t tier);
/* Where a unit sits: 1 = HBM, 2 = pinned host memory, 0 = not a movable
 * unit, -1 on error. Has no reference counterpart (the reference's Ant
 * bookkeeping tracks tiers on the engine side); for tests and monitoring. */
int cheetah_hip_unit_tier(const cheetah_hip_model *m, const char *unit_id);

/* ------------------------------------------------------------------------
 * Measurement hooks (events on the stream the kernels run on).
 * ---------------------------------------------------------------------- */
/* Times `iters` launches of one op-level GEMV over `nbuf` rotating weight
 * buffers (defeats the 256 MB Infinity Cache); returns the mean
 * milliseconds per launch in *ms. fmt: 1 = BF16, 4 = q8, 5 = q4. */
int cheetah_hip_time_gemv(uint32_t fmt, const void *const *w, size_t nbuf, size_t rows, size_t cols,
                          const float *x, float *y, size_t iters, float *ms);
/* Times `iters` launches of the op-level GEMM (n input rows) over `nbuf`
 * rotating weight buffers; mean milliseconds per launch in *ms. */
int cheetah_hip_time_gemm(uint32_t fmt, const void *const *w, size_t nbuf, size_t rows, size_t cols,
                          const float *x, size_t n, float *y, size_t iters, float *ms);
/* Times `iters` launches of cheetah_hip_attention over `nviews` rotating KV
 * caches (views[i]); mean milliseconds per launch in *ms. */
int cheetah_hip_time_attention(const float *q, const cheetah_hip_kv_view *views, size_t nviews, uint32_t q_heads,
                               size_t rows, size_t offset, float *out, size_t iters, float *ms);
/* Times `steps` greedy decode steps of a model already holding `offset`
 * cached positions (the decode graph replayed back to back), and the
 * model's largest GEMV alone over the same steps; both in ms per step. */
int cheetah_hip_time_decode(cheetah_hip_model *m, uint32_t token, size_t offset, size_t steps,
                            float *ms_per_step, float *gemv_ms_per_launch, uint32_t *tokens_out);

#ifdef __cplusplus
}
#endif

#endif
