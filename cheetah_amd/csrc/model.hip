// The HIP ModelForward (registry.rs:57-85) for the qwen2 / llama decoder
// forward (registrations/qwen2.rs:132-597, llama.rs:134-600).
//
// Device residency: every weight lives in HBM in the reference's own byte
// layout (BF16 rows; Q8/Q4 scale head + padded rows). q/k/v are stored as
// one [q_dim + 2 kv_dim, hidden] matrix (row-wise quantization makes
// quantize(concat) == concat(quantize)), gate and up stay separate matrices
// read by one dual GEMV / GEMM whose epilogue applies SwiGLU.
//
// KV cache: BF16 pages of 64 positions, [page][kv_head][64][head_dim] per
// layer for K and for V. A page id indexes every layer's pool; one page
// table per model maps logical page -> physical page. Pages are refcounted
// across a model, its clones and snapshots: a snapshot takes references, a
// restore maps them, and the first write into a shared page copies it.
//
// Decode (n == 1) is one captured hipGraph: embedding, 24-32 layers of
// {QKV GEMV with fused RMSNorm + bias, RoPE + KV append, split-K attention,
// o GEMV + residual, gate/up GEMV with fused RMSNorm + SwiGLU, down GEMV +
// residual}, LM head GEMV with fused final norm, argmax. The token and
// position live in device memory, so the same graph replays every step and
// the greedy loop can run back to back with no host round trip.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cheetah_hip.h"
#include "decode_fused.hpp"
#include "kernels.hpp"

namespace chip {
int ensure_ready();
}

using namespace chip;

namespace {

constexpr int kPageSize = 64;
constexpr int kPrefillSplits = 16;

struct DevAlloc {
    std::vector<void *> ptrs;
    template <class T>
    int alloc(T **p, size_t count) {
        void *q = nullptr;
        CHIP_CHECK(hipMalloc(&q, count * sizeof(T) > 0 ? count * sizeof(T) : 16));
        ptrs.push_back(q);
        *p = (T *)q;
        return 0;
    }
    void release(void *p) {
        for (auto &q : ptrs)
            if (q == p) {
                (void)hipFree(q);
                q = nullptr;
            }
    }
    ~DevAlloc() {
        for (void *q : ptrs)
            if (q) (void)hipFree(q);
    }
};

struct Staged {
    void *dev = nullptr;            // 2-D units: device BF16 copy
    std::vector<uint16_t> host;     // 1-D units: host BF16 copy
    std::vector<uint64_t> shape;
};

constexpr int kLayerMats = 5;  // qkv, o, gate, up, down

struct Layer {
    WMat qkv, o, gate, up, down;
    float *qkv_bias = nullptr;  // f32 [q_dim + 2 kv_dim] (zeros when absent)
    float *o_bias = nullptr;    // f32 [hidden] or null
    uint16_t *ln1 = nullptr, *ln2 = nullptr;
    KvLayer kv;
    // The persistent decode kernel's copy of down_proj, columns regrouped
    // per FFN block of the grid (fused_down_columns); built while down is
    // resident, freed when down is evicted to the host tier.
    uint16_t *down_cols = nullptr;
    // Host tier: pinned copy of a matrix whose device buffer was released
    // (its WMat base is then null); indexed like mat(). Null when resident.
    uint8_t *host[kLayerMats] = {};
    WMat &mat(int i) {
        WMat *w[] = {&qkv, &o, &gate, &up, &down};
        return *w[i];
    }
    const WMat &mat(int i) const { return const_cast<Layer *>(this)->mat(i); }
    bool streamed() const {
        for (const uint8_t *h : host)
            if (h) return true;
        return false;
    }
};

// Byte offset of matrix i in a feed slot (each matrix 256-byte aligned, the
// alignment of its own device buffer).
size_t slot_offset(const Layer &L, int i) {
    size_t off = 0;
    for (int j = 0; j < i; ++j) off += (L.mat(j).bytes() + 255) / 256 * 256;
    return off;
}

// Weights, rope table and KV pool: shared by a model, its clones and
// snapshots.
struct Shared {
    cheetah_hip_config cfg{};
    int quant = 0;  // 0, FMT_Q8, FMT_Q4
    int kv_f32 = 0;  // KV element type: 0 = BF16, 1 = f32
    size_t kv_capacity = 0, max_chunk = 0;
    bool finalized = false;
    std::unordered_map<std::string, Staged> staged;
    DevAlloc mem;
    std::vector<Layer> layers;
    uint16_t *embed = nullptr;
    WMat head;
    uint16_t *final_norm = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    int num_pages = 0;
    size_t page_elems = 0;  // elements of one page of one layer (K or V)
    size_t page_bytes() const { return page_elems * (kv_f32 ? 4 : 2); }
    std::mutex mu;
    std::vector<int> refs;
    std::vector<int> free_list;
    hipStream_t copy_stream = nullptr;
    int host_mats = 0;       // layer matrices on the host tier
    unsigned epoch = 0;      // bumped whenever a weight's device address changes
    // The layers' down_cols: built for down_cols_nf FFN blocks, generation
    // down_cols_gen (0: none; an eviction of a down_proj frees them).
    int down_cols_nf = 0;
    unsigned down_cols_gen = 0, down_cols_builds = 0;
    size_t slot_bytes = 0;   // one layer's matrices, as a feed slot holds them

    int q_dim() const { return (int)(cfg.q_heads * cfg.head_dim); }
    int kv_dim() const { return (int)(cfg.kv_heads * cfg.head_dim); }

    ~Shared() {
        if (copy_stream) {
            (void)hipStreamSynchronize(copy_stream);
            (void)hipStreamDestroy(copy_stream);
        }
        for (auto &kv : staged)
            if (kv.second.dev) (void)hipFree(kv.second.dev);
        for (Layer &L : layers)
            for (uint8_t *h : L.host)
                if (h) (void)hipHostFree(h);
    }

    int page_alloc() {
        std::lock_guard<std::mutex> lock(mu);
        if (free_list.empty()) return -1;
        int p = free_list.back();
        free_list.pop_back();
        refs[p] = 1;
        return p;
    }
    void page_ref(int p) {
        std::lock_guard<std::mutex> lock(mu);
        ++refs[p];
    }
    void page_unref(int p) {
        std::lock_guard<std::mutex> lock(mu);
        if (--refs[p] == 0) free_list.push_back(p);
    }
    int page_refs(int p) {
        std::lock_guard<std::mutex> lock(mu);
        return refs[p];
    }
};

}  // namespace

struct cheetah_hip_snapshot {
    std::shared_ptr<Shared> sh;
    std::vector<int> pages;
    size_t positions = 0;
    ~cheetah_hip_snapshot() {
        for (int p : pages) sh->page_unref(p);
    }
};

struct cheetah_hip_model {
    std::shared_ptr<Shared> sh;
    hipStream_t stream = nullptr;
    DevAlloc mem;
    std::vector<int> pages;  // logical -> physical
    std::vector<int32_t> page_host;
    int32_t *page_dev = nullptr;
    size_t len = 0;
    // activations
    float *hidden = nullptr, *normed = nullptr, *qkv = nullptr, *qrot = nullptr, *attn = nullptr, *act = nullptr;
    float *logits = nullptr, *part = nullptr;
    size_t part_floats = 0;
    float *gemm_ws = nullptr;  // split-K chunk sums of the prefill GEMMs
    size_t gemm_ws_floats = 0;
    uint16_t *xh = nullptr, *xl = nullptr;  // a GEMM input split into BF16 halves, [R][max width]
    uint16_t *ah = nullptr, *al = nullptr;  // the SwiGLU output as BF16 halves, [R][intermediate]
    uint32_t *tokens_dev = nullptr, *next_dev = nullptr, *hist_dev = nullptr;
    int32_t *step_dev = nullptr;  // [0] = token, [1] = position
    void *argmax_scratch = nullptr;
    int32_t *step_host = nullptr;    // pinned
    uint32_t *tokens_host = nullptr;  // pinned staging for chunk tokens
    float *logits_host = nullptr;     // pinned
    // Decode graphs, one per attention split count (the grid of a captured
    // launch is fixed; the split count follows the context length).
    std::vector<hipGraphExec_t> graphs = std::vector<hipGraphExec_t>(attention_max_splits() + 1, nullptr);
    // Persistent decode kernel state (decode_fused.hip).
    bool fused_ok = false;
    FusedLayer *fused_layers = nullptr;  // device [L]
    unsigned table_cols_gen = 0;         // generation of the down_cols the table points at (0: none yet)
    int fused_blocks = 0;
    FusedGeom fused_geo{};               // role geometry on fused_blocks blocks
    uint64_t *tagged = nullptr;  // hid0 | hid1 | kvw | part | ml | pdown | am, tagged words
    size_t tagged_words = 0;
    int32_t *abort_dev = nullptr;
    unsigned next_tag = 1;          // tag of the next launch's first phase
    int32_t *abort_host = nullptr;  // pinned
    unsigned epoch = 0;             // the weight epoch the graphs and layer table were built for
    // Host-tier feed: layer l's streamed matrices are copied from pinned
    // host memory into slot l % 2 on feed_stream, one streamed layer ahead
    // of the compute stream. ready[k] marks a finished copy into slot k,
    // released[k] the end of the last kernel reading it; fed[k] is the
    // layer rebased onto the slot.
    hipStream_t feed_stream = nullptr;
    uint8_t *slot[2] = {};
    int slot_layer[2] = {-1, -1};
    unsigned slot_epoch[2] = {};
    hipEvent_t ready[2] = {}, released[2] = {};
    Layer fed[2];

    ~cheetah_hip_model() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (feed_stream) {
            (void)hipStreamSynchronize(feed_stream);
            (void)hipStreamDestroy(feed_stream);
        }
        for (int k = 0; k < 2; ++k) {
            if (ready[k]) (void)hipEventDestroy(ready[k]);
            if (released[k]) (void)hipEventDestroy(released[k]);
        }
        for (hipGraphExec_t g : graphs)
            if (g) (void)hipGraphExecDestroy(g);
        if (stream) (void)hipStreamDestroy(stream);
        if (step_host) (void)hipHostFree(step_host);
        if (tokens_host) (void)hipHostFree(tokens_host);
        if (logits_host) (void)hipHostFree(logits_host);
        if (abort_host) (void)hipHostFree(abort_host);
        for (int p : pages) sh->page_unref(p);
    }
};

namespace {

const cheetah_hip_config &C(const cheetah_hip_model *m) { return m->sh->cfg; }

int upload_bf16_1d(Shared &sh, const std::string &id, size_t expect, uint16_t **out, bool required) {
    auto it = sh.staged.find(id);
    if (it == sh.staged.end()) {
        if (required) return fail("HIP backend: missing unit '" + id + "'.");
        *out = nullptr;
        return 0;
    }
    if (it->second.host.size() != expect)
        return fail("HIP backend: unit '" + id + "' has " + std::to_string(it->second.host.size()) +
                    " elements, expected " + std::to_string(expect) + ".");
    CHIP_TRY(sh.mem.alloc(out, expect));
    CHIP_CHECK(hipMemcpy(*out, it->second.host.data(), expect * 2, hipMemcpyHostToDevice));
    return 0;
}

// Bias units widened to f32 on the host (bias adds are v + bf16_f32(b),
// ops.rs:1156-1166); absent units become zeros (unit-optional adds).
int append_bias(Shared &sh, const std::string &id, size_t n, std::vector<float> &out) {
    auto it = sh.staged.find(id);
    if (it == sh.staged.end()) {
        out.insert(out.end(), n, 0.0f);
        return 0;
    }
    if (it->second.host.size() != n) return fail("HIP backend: bias unit '" + id + "' has the wrong length.");
    for (uint16_t b : it->second.host) {
        uint32_t u = (uint32_t)b << 16;
        float f;
        std::memcpy(&f, &u, 4);
        out.push_back(f);
    }
    return 0;
}

int take_2d(Shared &sh, const std::string &id, size_t rows, size_t cols, void **dev) {
    auto it = sh.staged.find(id);
    if (it == sh.staged.end() || !it->second.dev) return fail("HIP backend: missing unit '" + id + "'.");
    const auto &s = it->second.shape;
    if (s.size() != 2 || s[0] != rows || s[1] != cols)
        return fail("Linear unit '" + id + "' does not match its " + std::to_string(rows) + "x" +
                    std::to_string(cols) + " shape.");
    *dev = it->second.dev;
    it->second.dev = nullptr;
    return 0;
}

// BF16 device matrix -> the model's linear format (quantized when selected).
int make_linear(Shared &sh, void *bf16, size_t rows, size_t cols, WMat *out) {
    if (!sh.quant) {
        sh.mem.ptrs.push_back(bf16);
        *out = WMat{FMT_BF16, (const uint8_t *)bf16, rows, cols};
        return 0;
    }
    uint8_t *q = nullptr;
    CHIP_TRY(sh.mem.alloc(&q, fmt_buffer_bytes(sh.quant, rows, cols)));
    CHIP_TRY(launch_quantize(sh.quant, (const uint16_t *)bf16, rows, cols, q, sh.copy_stream));
    CHIP_CHECK(hipStreamSynchronize(sh.copy_stream));
    CHIP_CHECK(hipFree(bf16));
    *out = WMat{sh.quant, q, rows, cols};
    return 0;
}

int finalize(cheetah_hip_model *m) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    const size_t H = c.hidden_size, qd = sh.q_dim(), kvd = sh.kv_dim(), I = c.intermediate_size, V = c.vocab_size;
    CHIP_CHECK(hipStreamCreateWithFlags(&sh.copy_stream, hipStreamNonBlocking));
    // Embedding and head (BF16, never quantized: ops.rs:1533-1537).
    void *emb = nullptr;
    CHIP_TRY(take_2d(sh, "model.embed_tokens.weight", V, H, &emb));
    sh.mem.ptrs.push_back(emb);
    sh.embed = (uint16_t *)emb;
    if (c.tie_word_embeddings) {
        sh.head = WMat{FMT_BF16, (const uint8_t *)emb, V, H};
    } else {
        void *head = nullptr;
        if (take_2d(sh, "lm_head.weight", V, H, &head))
            return fail("Native backend: neither tied embeddings nor a separate 'lm_head.weight' tensor are present.");
        sh.mem.ptrs.push_back(head);
        sh.head = WMat{FMT_BF16, (const uint8_t *)head, V, H};
    }
    CHIP_TRY(upload_bf16_1d(sh, "model.norm.weight", H, &sh.final_norm, true));
    sh.layers.resize(c.num_layers);
    std::vector<int32_t> perm(qd + 2 * kvd);
    for (size_t r = 0; r < perm.size(); ++r)
        perm[r] = qkv_perm_row((int)r, (int)c.q_heads, (int)c.kv_heads, (int)c.head_dim, (int)c.rotary_dim);
    int32_t *perm_dev = nullptr;
    CHIP_TRY(sh.mem.alloc(&perm_dev, perm.size()));
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        Layer &L = sh.layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        CHIP_TRY(upload_bf16_1d(sh, p + "input_layernorm.weight", H, &L.ln1, true));
        CHIP_TRY(upload_bf16_1d(sh, p + "post_attention_layernorm.weight", H, &L.ln2, true));
        void *q = nullptr, *k = nullptr, *v = nullptr;
        CHIP_TRY(take_2d(sh, p + "self_attn.q_proj.weight", qd, H, &q));
        CHIP_TRY(take_2d(sh, p + "self_attn.k_proj.weight", kvd, H, &k));
        CHIP_TRY(take_2d(sh, p + "self_attn.v_proj.weight", kvd, H, &v));
        uint16_t *qkv = nullptr;
        CHIP_CHECK(hipMalloc(&qkv, (qd + 2 * kvd) * H * 2));
        CHIP_CHECK(hipMemcpyAsync(qkv, q, qd * H * 2, hipMemcpyDeviceToDevice, sh.copy_stream));
        CHIP_CHECK(hipMemcpyAsync(qkv + qd * H, k, kvd * H * 2, hipMemcpyDeviceToDevice, sh.copy_stream));
        CHIP_CHECK(hipMemcpyAsync(qkv + (qd + kvd) * H, v, kvd * H * 2, hipMemcpyDeviceToDevice, sh.copy_stream));
        // Pair-permute the q/k rows so each RoPE pair is two adjacent rows
        // (qkv_perm_row); quantization below is per row, so it commutes.
        uint16_t *qkv_p = nullptr;
        CHIP_CHECK(hipMalloc(&qkv_p, (qd + 2 * kvd) * H * 2));
        CHIP_CHECK(hipMemcpyAsync(perm_dev, perm.data(), perm.size() * 4, hipMemcpyHostToDevice, sh.copy_stream));
        CHIP_TRY(launch_gather_rows((const uint8_t *)qkv, (uint8_t *)qkv_p, perm_dev, qd + 2 * kvd, H * 2,
                                    sh.copy_stream));
        CHIP_CHECK(hipStreamSynchronize(sh.copy_stream));
        CHIP_CHECK(hipFree(q));
        CHIP_CHECK(hipFree(k));
        CHIP_CHECK(hipFree(v));
        CHIP_CHECK(hipFree(qkv));
        CHIP_TRY(make_linear(sh, qkv_p, qd + 2 * kvd, H, &L.qkv));
        std::vector<float> bias_ref, bias;
        CHIP_TRY(append_bias(sh, p + "self_attn.q_proj.bias", qd, bias_ref));
        CHIP_TRY(append_bias(sh, p + "self_attn.k_proj.bias", kvd, bias_ref));
        CHIP_TRY(append_bias(sh, p + "self_attn.v_proj.bias", kvd, bias_ref));
        for (int32_t r : perm) bias.push_back(bias_ref[r]);
        CHIP_TRY(sh.mem.alloc(&L.qkv_bias, bias.size()));
        CHIP_CHECK(hipMemcpy(L.qkv_bias, bias.data(), bias.size() * 4, hipMemcpyHostToDevice));
        if (sh.staged.count(p + "self_attn.o_proj.bias")) {
            std::vector<float> ob;
            CHIP_TRY(append_bias(sh, p + "self_attn.o_proj.bias", H, ob));
            CHIP_TRY(sh.mem.alloc(&L.o_bias, H));
            CHIP_CHECK(hipMemcpy(L.o_bias, ob.data(), H * 4, hipMemcpyHostToDevice));
        }
        void *o = nullptr, *g = nullptr, *u = nullptr, *d = nullptr;
        CHIP_TRY(take_2d(sh, p + "self_attn.o_proj.weight", H, qd, &o));
        CHIP_TRY(take_2d(sh, p + "mlp.gate_proj.weight", I, H, &g));
        CHIP_TRY(take_2d(sh, p + "mlp.up_proj.weight", I, H, &u));
        CHIP_TRY(take_2d(sh, p + "mlp.down_proj.weight", H, I, &d));
        CHIP_TRY(make_linear(sh, o, H, qd, &L.o));
        CHIP_TRY(make_linear(sh, g, I, H, &L.gate));
        CHIP_TRY(make_linear(sh, u, I, H, &L.up));
        CHIP_TRY(make_linear(sh, d, H, I, &L.down));
    }
    for (auto &kv : sh.staged)
        if (kv.second.dev) {
            (void)hipFree(kv.second.dev);
            kv.second.dev = nullptr;
        }
    sh.staged.clear();
    sh.slot_bytes = slot_offset(sh.layers[0], kLayerMats);  // every layer has the same shapes

    // RoPE table: angle = pos * theta^(-2i/rotary_dim), with libm powf/sinf/
    // cosf exactly as rope_in_place computes it (ops.rs:702-707).
    const size_t half = c.rotary_dim / 2;
    std::vector<float> cs(sh.kv_capacity * half), sn(sh.kv_capacity * half);
    std::vector<float> freq(half);
    for (size_t i = 0; i < half; ++i) freq[i] = powf(c.rope_theta, -2.0f * (float)i / (float)c.rotary_dim);
    for (size_t pos = 0; pos < sh.kv_capacity; ++pos)
        for (size_t i = 0; i < half; ++i) {
            const float angle = (float)pos * freq[i];
            sn[pos * half + i] = sinf(angle);
            cs[pos * half + i] = cosf(angle);
        }
    CHIP_TRY(sh.mem.alloc(&sh.rope_cos, cs.size()));
    CHIP_TRY(sh.mem.alloc(&sh.rope_sin, sn.size()));
    CHIP_CHECK(hipMemcpy(sh.rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    CHIP_CHECK(hipMemcpy(sh.rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));

    // KV pool.
    sh.num_pages = (int)((sh.kv_capacity + kPageSize - 1) / kPageSize);
    sh.page_elems = (size_t)c.kv_heads * kPageSize * c.head_dim;
    for (auto &L : sh.layers) {
        uint8_t *k = nullptr, *v = nullptr;
        CHIP_TRY(sh.mem.alloc(&k, sh.page_bytes() * sh.num_pages));
        CHIP_TRY(sh.mem.alloc(&v, sh.page_bytes() * sh.num_pages));
        L.kv.k = k;
        L.kv.v = v;
    }
    sh.refs.assign(sh.num_pages, 0);
    sh.free_list.clear();
    for (int p = sh.num_pages - 1; p >= 0; --p) sh.free_list.push_back(p);
    sh.finalized = true;
    return 0;
}

// Sizes (words) of the tagged arrays in one allocation: hid0, hid1, kvw,
// part, ml, pdown, am; each rounded to an even count plus 2 words, so every array
// starts 16-byte aligned and a 16-byte read at its last word stays inside.
std::vector<size_t> fused_tagged_sizes(const cheetah_hip_model *m) {
    const auto &c = m->sh->cfg;
    const FusedGeom &g = m->fused_geo;
    const size_t raw[] = {c.hidden_size, c.hidden_size, c.kv_heads * 2 * c.head_dim,
                          (size_t)g.no * g.ni_max * 8, 2 * (size_t)g.ni_max, (size_t)g.no * g.nbd * 8,
                          4 * (size_t)m->fused_blocks};
    std::vector<size_t> out;
    for (size_t n : raw) out.push_back((n + 1) / 2 * 2 + 2);
    return out;
}

// The persistent kernel's per-layer pointer table (device addresses of the
// weights as they are now; a host-tier matrix has none and the kernel is not
// used while one exists).
int upload_fused_layers(cheetah_hip_model *m) {
    const Shared &sh = *m->sh;
    std::vector<FusedLayer> fl(sh.cfg.num_layers);
    for (uint32_t l = 0; l < sh.cfg.num_layers; ++l) {
        const Layer &L = sh.layers[l];
        fl[l] = FusedLayer{L.qkv.payload(), L.o.payload(), L.gate.payload(), L.up.payload(), L.down.payload(),
                           L.qkv.scales(), L.o.scales(), L.gate.scales(), L.up.scales(), L.down.scales(),
                           L.qkv_bias, L.o_bias, L.ln1, L.ln2, L.kv.k, L.kv.v, L.down_cols};
    }
    CHIP_CHECK(hipMemcpy(m->fused_layers, fl.data(), fl.size() * sizeof(FusedLayer), hipMemcpyHostToDevice));
    return 0;
}

int ensure_down_cols(cheetah_hip_model *m);

// Persistent decode state of one instance: the per-layer pointer table and
// the tagged hand-off words. Sets fused_ok when the model's shape and layout
// have a persistent kernel; otherwise decode keeps the graph path.
int init_fused(cheetah_hip_model *m) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    const Layer &L0 = sh.layers[0];
    auto aligned = [](const WMat &w) { return w.row_stride() % 16 == 0 && ((uintptr_t)w.payload() % 16) == 0; };
    // The persistent kernel reads weight rows in 16-byte units through buffer
    // resources (byte ranges below 2 GiB) and copies the embedding row and the
    // RMSNorm gains into LDS 16 bytes at a time.
    auto a16 = [](const void *p) { return (uintptr_t)p % 16 == 0; };
    auto fits = [](const WMat &w, size_t rows) { return rows * w.row_stride() < (size_t(1) << 31); };
    const size_t qkv_rows = c.q_heads * c.head_dim + 2 * c.kv_heads * c.head_dim;
    bool al = a16(sh.head.base) && a16(sh.embed) && a16(sh.final_norm) &&
              (size_t)c.vocab_size * c.hidden_size * 2 < (size_t(1) << 31);
    for (const Layer &L : sh.layers)
        al = al && aligned(L.qkv) && aligned(L.o) && aligned(L.gate) && aligned(L.up) && aligned(L.down) &&
             a16(L.ln1) && a16(L.ln2) && fits(L.qkv, qkv_rows) && fits(L.o, c.hidden_size) &&
             fits(L.gate, c.intermediate_size) && fits(L.up, c.intermediate_size) && fits(L.down, c.hidden_size);
    m->fused_blocks = fused_decode_blocks();
    // The kernel addresses one layer's K (or V) pool with 30-bit element
    // indices.
    const bool small_pool = (size_t)sh.num_pages * c.kv_heads * kPageSize * c.head_dim < (size_t(1) << 30);
    m->fused_ok = small_pool && fused_decode_supported(L0.qkv.fmt, (int)c.hidden_size, (int)c.q_heads,
                                                       (int)c.kv_heads, (int)c.head_dim, (int)c.intermediate_size,
                                                       al, m->fused_blocks);
    if (!m->fused_ok) return 0;
    m->fused_geo = fused_geometry((int)c.hidden_size, (int)c.q_heads, (int)c.kv_heads, (int)c.head_dim,
                                  (int)c.intermediate_size, sh.kv_f32 != 0, m->fused_blocks);
    CHIP_TRY(m->mem.alloc(&m->fused_layers, c.num_layers));
    CHIP_TRY(upload_fused_layers(m));
    if (!sh.host_mats) CHIP_TRY(ensure_down_cols(m));
    m->tagged_words = 0;
    for (size_t n : fused_tagged_sizes(m)) m->tagged_words += n;
    CHIP_TRY(m->mem.alloc(&m->tagged, m->tagged_words));
    CHIP_CHECK(hipMemset(m->tagged, 0, m->tagged_words * sizeof(uint64_t)));
    CHIP_TRY(m->mem.alloc(&m->abort_dev, 1));
    CHIP_CHECK(hipMemset(m->abort_dev, 0, sizeof(int32_t)));
    m->next_tag = 1;
    CHIP_CHECK(hipHostMalloc((void **)&m->abort_host, sizeof(int32_t), hipHostMallocDefault));
    return 0;
}

bool fused_enabled(const cheetah_hip_model *m) {
    if (!m->fused_ok) return false;
    // CHEETAH_HIP_FUSED=0 selects the per-step graph path instead.
    const char *e = getenv("CHEETAH_HIP_FUSED");
    return !(e && (e[0] == '0' || e[0] == 'f' || e[0] == 'F' || e[0] == 'n' || e[0] == 'N'));
}

// Whether one persistent launch can run decode steps at positions
// [offset, offset + steps): the attention runs of the longest context must
// fit the item blocks.
bool fused_fits(const cheetah_hip_model *m, size_t offset, size_t steps) {
    // The persistent kernel reads every layer from HBM in place.
    if (!fused_enabled(m) || m->sh->host_mats) return false;
    return (long)(offset + steps) <= fused_max_context(m->fused_geo);
}

// Builds every layer's down_cols for the FFN blocks of this instance's grid
// once per model (the persistent kernel runs only while every matrix is
// resident; an eviction of a down_proj frees them and they are rebuilt
// here), and points this instance's layer table at them.
int ensure_down_cols(cheetah_hip_model *m) {
    Shared &sh = *m->sh;
    {
        std::lock_guard<std::mutex> lock(sh.mu);
        const int nf = m->fused_geo.nf;
        if (sh.down_cols_gen != 0 && sh.down_cols_nf != nf) return fail("HIP backend: persistent decode grid changed.");
        if (sh.down_cols_gen == 0) {
            const auto &c = sh.cfg;
            const int H = (int)c.hidden_size, I = (int)c.intermediate_size;
            const size_t elems = (size_t)nf * H * fused_gate_rows_padded(I, nf);
            for (Layer &L : sh.layers) {
                if (!L.down.payload()) return fail("HIP backend: persistent decode needs every matrix resident.");
                if (!L.down_cols) CHIP_TRY(sh.mem.alloc(&L.down_cols, elems));
                CHIP_TRY(fused_down_columns((const uint16_t *)L.down.payload(), L.down.row_stride(), H, I, nf,
                                            L.down_cols, m->stream));
            }
            CHIP_CHECK(hipStreamSynchronize(m->stream));
            sh.down_cols_nf = nf;
            sh.down_cols_gen = ++sh.down_cols_builds;
        }
        if (m->table_cols_gen == sh.down_cols_gen) return 0;
        m->table_cols_gen = sh.down_cols_gen;
    }
    return upload_fused_layers(m);
}

// Runs `steps` decode steps in one persistent launch from the token and
// position (`offset`, also in step_dev); leaves the last step's logits in
// m->logits, its argmax in next_dev and every sampled id in hist_dev. Waits
// for the launch.
int run_fused(cheetah_hip_model *m, size_t offset, size_t steps) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    CHIP_TRY(ensure_down_cols(m));
    const unsigned per_step = (unsigned)fused_phases_per_step((int)c.num_layers);
    if ((uint64_t)m->next_tag + (uint64_t)steps * per_step >= 0xFFFFFF00ull) {
        // Tags are about to wrap: start over from zeroed words.
        CHIP_CHECK(hipMemsetAsync(m->tagged, 0, m->tagged_words * sizeof(uint64_t), m->stream));
        m->next_tag = 1;
    }
    FusedArgs a{};
    a.layers = m->fused_layers;
    a.L = (int)c.num_layers;
    a.H = (int)c.hidden_size;
    a.q_heads = (int)c.q_heads;
    a.kv_heads = (int)c.kv_heads;
    a.rotary = (int)c.rotary_dim;
    a.I = (int)c.intermediate_size;
    a.V = (int)c.vocab_size;
    a.eps = c.rms_eps;
    const Layer &L0 = sh.layers[0];
    a.qkv_stride = L0.qkv.row_stride();
    a.o_stride = L0.o.row_stride();
    a.gu_stride = L0.gate.row_stride();
    a.down_stride = L0.down.row_stride();
    a.embed = sh.embed;
    a.head = (const uint16_t *)sh.head.base;
    a.final_norm = sh.final_norm;
    a.rope_cos = sh.rope_cos;
    a.rope_sin = sh.rope_sin;
    a.page_table = m->page_dev;
    a.step = m->step_dev;
    a.hist = m->hist_dev;
    a.hist_cap = (long)sh.kv_capacity + 1;
    a.logits = m->logits;
    uint64_t *t = m->tagged;
    uint64_t **dst[] = {&a.hid0, &a.hid1, &a.kvw, &a.part, &a.ml, &a.pdown, &a.am};
    const std::vector<size_t> sizes = fused_tagged_sizes(m);
    for (size_t i = 0; i < sizes.size(); ++i) {
        *dst[i] = t;
        t += sizes[i];
    }
    a.abort_flag = m->abort_dev;
    a.tag0 = m->next_tag;
    a.steps = (int)steps;
    a.ctx_end = (long)(offset + steps);
    // CHEETAH_HIP_FUSED_TRACE=<file>: per-phase timestamps of the launch's
    // last step, one line per block (wall clock ticks).
    const char *trace_path = getenv("CHEETAH_HIP_FUSED_TRACE");
    const size_t trace_events = 16 * (size_t)c.num_layers + 3;
    if (trace_path && *trace_path) {
        CHIP_CHECK(hipMalloc((void **)&a.trace, (size_t)m->fused_blocks * trace_events * sizeof(uint64_t)));
        CHIP_CHECK(hipMemsetAsync(a.trace, 0, (size_t)m->fused_blocks * trace_events * sizeof(uint64_t), m->stream));
        a.trace_step = (int)steps - 1;
    }
    CHIP_TRY(launch_decode_fused(a, L0.qkv.fmt, (int)c.head_dim, (int)(c.q_heads / c.kv_heads), sh.kv_f32 != 0,
                                 m->stream));
    if (a.trace) {
        std::vector<uint64_t> tr((size_t)m->fused_blocks * trace_events);
        CHIP_CHECK(hipMemcpyAsync(tr.data(), a.trace, tr.size() * sizeof(uint64_t), hipMemcpyDeviceToHost, m->stream));
        CHIP_CHECK(hipStreamSynchronize(m->stream));
        CHIP_CHECK(hipFree(a.trace));
        if (FILE *f = fopen(trace_path, "w")) {
            for (int blk = 0; blk < m->fused_blocks; ++blk) {
                for (size_t e = 0; e < trace_events; ++e) fprintf(f, e ? " %llu" : "%llu", (unsigned long long)tr[blk * trace_events + e]);
                fprintf(f, "\n");
            }
            fclose(f);
        }
    }
    m->next_tag += (unsigned)steps * per_step;
    CHIP_CHECK(hipMemcpyAsync(m->next_dev, m->step_dev, sizeof(uint32_t), hipMemcpyDeviceToDevice, m->stream));
    CHIP_CHECK(hipMemcpyAsync(m->abort_host, m->abort_dev, sizeof(int32_t), hipMemcpyDeviceToHost, m->stream));
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    if (*m->abort_host) {
        // A poll timed out: the steps are incomplete. Reset the hand-off
        // words so the next launch starts clean.
        CHIP_CHECK(hipMemset(m->tagged, 0, m->tagged_words * sizeof(uint64_t)));
        CHIP_CHECK(hipMemset(m->abort_dev, 0, sizeof(int32_t)));
        m->next_tag = 1;
        return fail("HIP backend: persistent decode timed out waiting for its inputs; the steps were abandoned.");
    }
    return 0;
}

// Per-instance buffers (a fresh model and every clone).
int init_instance(cheetah_hip_model *m) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    const size_t H = c.hidden_size, qd = sh.q_dim(), kvd = sh.kv_dim(), R = sh.max_chunk;
    CHIP_CHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    CHIP_CHECK(hipStreamCreateWithFlags(&m->feed_stream, hipStreamNonBlocking));
    for (int k = 0; k < 2; ++k) {
        CHIP_CHECK(hipEventCreateWithFlags(&m->ready[k], hipEventDisableTiming));
        CHIP_CHECK(hipEventCreateWithFlags(&m->released[k], hipEventDisableTiming));
        CHIP_CHECK(hipEventRecord(m->released[k], m->stream));
    }
    m->epoch = sh.epoch;
    CHIP_TRY(m->mem.alloc(&m->hidden, R * H));
    CHIP_TRY(m->mem.alloc(&m->normed, R * H));
    CHIP_TRY(m->mem.alloc(&m->qkv, R * (qd + 2 * kvd)));
    CHIP_TRY(m->mem.alloc(&m->attn, R * qd));
    CHIP_TRY(m->mem.alloc(&m->qrot, R * qd));
    CHIP_TRY(m->mem.alloc(&m->act, R * c.intermediate_size));
    CHIP_TRY(m->mem.alloc(&m->logits, c.vocab_size));
    // Prefill partials: the fixed VALU split count, or the matrix-core
    // kernel's span splits at full capacity; decode: attention_max_splits.
    const size_t prefill_splits =
        std::max((size_t)kPrefillSplits,
                 (size_t)attention_prefill_splits(sh.kv_capacity, attention_prefill_span(sh.kv_capacity)));
    const size_t part_rows = std::max(R * prefill_splits, (size_t)attention_max_splits());
    m->part_floats = part_rows * c.q_heads * (c.head_dim + 2);
    CHIP_TRY(m->mem.alloc(&m->part, m->part_floats));
    {
        const size_t qd = sh.q_dim(), kvd = sh.kv_dim(), I = c.intermediate_size, H = c.hidden_size;
        m->gemm_ws_floats = std::max({gemm_split_workspace_floats(qd + 2 * kvd, H, R, false),
                                      gemm_split_workspace_floats(H, qd, R, false),
                                      gemm_split_workspace_floats(I, H, R, true),
                                      gemm_split_workspace_floats(H, I, R, false), (size_t)1});
        CHIP_TRY(m->mem.alloc(&m->gemm_ws, m->gemm_ws_floats));
        const size_t width = std::max({H, qd, I});
        CHIP_TRY(m->mem.alloc(&m->xh, R * width));
        CHIP_TRY(m->mem.alloc(&m->xl, R * width));
        CHIP_TRY(m->mem.alloc(&m->ah, R * I));
        CHIP_TRY(m->mem.alloc(&m->al, R * I));
    }
    CHIP_TRY(m->mem.alloc(&m->tokens_dev, sh.kv_capacity));
    CHIP_TRY(m->mem.alloc(&m->next_dev, 1));
    CHIP_TRY(m->mem.alloc(&m->hist_dev, sh.kv_capacity + 1));
    CHIP_TRY(m->mem.alloc(&m->step_dev, 2));
    uint8_t *scratch = nullptr;
    CHIP_TRY(m->mem.alloc(&scratch, argmax_scratch_bytes()));
    m->argmax_scratch = scratch;
    CHIP_TRY(m->mem.alloc(&m->page_dev, (size_t)sh.num_pages));
    CHIP_CHECK(hipHostMalloc((void **)&m->step_host, 2 * sizeof(int32_t), hipHostMallocDefault));
    CHIP_CHECK(hipHostMalloc((void **)&m->tokens_host, sh.kv_capacity * sizeof(uint32_t), hipHostMallocDefault));
    CHIP_CHECK(hipHostMalloc((void **)&m->logits_host, (size_t)c.vocab_size * sizeof(float), hipHostMallocDefault));
    m->page_host.assign(sh.num_pages, 0);
    return init_fused(m);
}

// Makes positions [m->len, m->len + n) writable: maps new pages and copies a
// shared page before its first write. Uploads the page table if it changed.
// All or nothing: when the pool runs out part way, every page this call
// copied or mapped is given back and the instance's page list is restored,
// so the host list, the device table and the reference counts stay as they
// were before the call (a later call maps the same positions afresh).
int reserve_positions(cheetah_hip_model *m, size_t n) {
    Shared &sh = *m->sh;
    const size_t end = m->len + n;
    if (end > sh.kv_capacity)
        return fail("HIP backend: KV cache capacity of " + std::to_string(sh.kv_capacity) +
                    " positions exceeded (needs " + std::to_string(end) + ").");
    // What this call changed: (logical page, page it replaced or -1 for a
    // page appended, page it mapped). A replaced shared page keeps this
    // instance's reference until the copies reading it have finished:
    // released earlier, another holder could see itself as the only one and
    // write the page in place while the copy still reads it.
    struct Change {
        size_t lp;
        int old_page, new_page;
    };
    std::vector<Change> log;
    auto roll_back = [&]() {
        // The copies into the new pages finish before those pages return to
        // the pool (a clone on another stream could be handed one at once).
        const hipError_t e = hipStreamSynchronize(m->stream);
        for (auto it = log.rbegin(); it != log.rend(); ++it) {
            if (it->old_page < 0) m->pages.pop_back();
            else m->pages[it->lp] = it->old_page;
            if (e == hipSuccess) sh.page_unref(it->new_page);
        }
        if (e != hipSuccess) return fail(std::string("HIP backend: ") + hipGetErrorString(e));
        return fail("HIP backend: KV page pool exhausted.");
    };
    const size_t first = m->len / kPageSize, last = (end - 1) / kPageSize;
    for (size_t lp = first; lp <= last; ++lp) {
        if (lp < m->pages.size()) {
            const int p = m->pages[lp];
            if (sh.page_refs(p) > 1) {  // copy on write
                const int np = sh.page_alloc();
                if (np < 0) return roll_back();
                for (auto &L : sh.layers) {
                    const size_t pb = sh.page_bytes();
                    uint8_t *k = (uint8_t *)L.kv.k, *v = (uint8_t *)L.kv.v;
                    CHIP_CHECK(hipMemcpyAsync(k + (size_t)np * pb, k + (size_t)p * pb, pb, hipMemcpyDeviceToDevice,
                                              m->stream));
                    CHIP_CHECK(hipMemcpyAsync(v + (size_t)np * pb, v + (size_t)p * pb, pb, hipMemcpyDeviceToDevice,
                                              m->stream));
                }
                log.push_back({lp, p, np});
                m->pages[lp] = np;
            }
        } else {
            const int np = sh.page_alloc();
            if (np < 0) return roll_back();
            log.push_back({lp, -1, np});
            m->pages.push_back(np);
        }
    }
    if (log.empty()) return 0;
    for (size_t i = 0; i < m->pages.size(); ++i) m->page_host[i] = m->pages[i];
    CHIP_CHECK(hipMemcpyAsync(m->page_dev, m->page_host.data(), m->pages.size() * sizeof(int32_t),
                              hipMemcpyHostToDevice, m->stream));
    CHIP_CHECK(hipStreamSynchronize(m->stream));  // page_host is pageable; the copies have finished
    for (const Change &c : log)
        if (c.old_page >= 0) sh.page_unref(c.old_page);
    return 0;
}

KvGeom geom(const cheetah_hip_model *m) {
    return KvGeom{m->page_dev, kPageSize, (int)C(m).kv_heads, (int)C(m).head_dim, m->sh->kv_f32};
}

// Copies layer l's host-tier matrices into slot l % 2 on the feed stream,
// after the last kernel that read the slot, and rebases fed[l % 2] onto it.
int feed_issue(cheetah_hip_model *m, uint32_t l) {
    Shared &sh = *m->sh;
    const int k = (int)(l & 1);
    if (!m->slot[k]) CHIP_TRY(m->mem.alloc(&m->slot[k], sh.slot_bytes));
    const Layer &src = sh.layers[l];
    Layer &dst = m->fed[k];
    dst = src;
    CHIP_CHECK(hipStreamWaitEvent(m->feed_stream, m->released[k], 0));
    for (int i = 0; i < kLayerMats; ++i) {
        if (!src.host[i]) continue;
        uint8_t *at = m->slot[k] + slot_offset(src, i);
        CHIP_CHECK(hipMemcpyAsync(at, src.host[i], src.mat(i).bytes(), hipMemcpyHostToDevice, m->feed_stream));
        dst.mat(i).base = at;
    }
    CHIP_CHECK(hipEventRecord(m->ready[k], m->feed_stream));
    m->slot_layer[k] = (int)l;
    m->slot_epoch[k] = sh.epoch;
    return 0;
}

bool slot_holds(const cheetah_hip_model *m, uint32_t l) {
    const int k = (int)(l & 1);
    return m->slot_layer[k] == (int)l && m->slot_epoch[k] == m->sh->epoch;
}

// The layer as the kernels enqueued next read it: the shared layer when all
// of its matrices are resident, else its copy rebased onto the feed slot,
// with the compute stream waiting for the slot's copy.
int layer_begin(cheetah_hip_model *m, uint32_t l, hipStream_t s, const Layer **out) {
    const Layer &L = m->sh->layers[l];
    *out = &L;
    if (!L.streamed()) return 0;
    if (!slot_holds(m, l)) CHIP_TRY(feed_issue(m, l));
    CHIP_CHECK(hipStreamWaitEvent(s, m->ready[l & 1], 0));
    *out = &m->fed[l & 1];
    return 0;
}

// After layer l's kernels: releases its slot and starts the copy of the next
// streamed layer (wrapping to the first one, for the next step), so the
// transfer overlaps the compute in between. A slot that already holds its
// layer is kept, so two streamed layers of different parity stay in place.
int layer_end(cheetah_hip_model *m, uint32_t l, hipStream_t s) {
    const Shared &sh = *m->sh;
    if (!sh.host_mats) return 0;
    if (sh.layers[l].streamed()) CHIP_CHECK(hipEventRecord(m->released[l & 1], s));
    const uint32_t n = sh.cfg.num_layers;
    for (uint32_t d = 1; d <= n; ++d) {
        const uint32_t next = (l + d) % n;
        if (!sh.layers[next].streamed()) continue;
        if (!slot_holds(m, next)) CHIP_TRY(feed_issue(m, next));
        break;
    }
    return 0;
}

// Brings an instance up to the current weight epoch: captured graphs and the
// persistent kernel's table hold device addresses that page_in / evict have
// changed.
int refresh_weights(cheetah_hip_model *m) {
    const Shared &sh = *m->sh;
    if (m->epoch == sh.epoch) return 0;
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    for (hipGraphExec_t &g : m->graphs)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    if (m->fused_ok && !sh.host_mats) CHIP_TRY(upload_fused_layers(m));
    m->epoch = sh.epoch;
    return 0;
}

// Attention splits of a decode step over `ctx` keys (one captured graph per
// split count).
int decode_splits(const cheetah_hip_model *m, size_t ctx) {
    return attention_decode_splits(ctx, (int)m->sh->cfg.kv_heads, 1, m->sh->kv_f32 != 0);
}

// One decode step's kernels; token and position are read from step_dev.
int enqueue_decode(cheetah_hip_model *m, int splits) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    hipStream_t s = m->stream;
    const int32_t *pos = m->step_dev + 1;
    CHIP_TRY(launch_embed(sh.embed, c.hidden_size, (const uint32_t *)m->step_dev, 1, m->hidden, s));
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const Layer *Lp = nullptr;
        CHIP_TRY(layer_begin(m, l, s, &Lp));
        const Layer &L = *Lp;
        GemvJob qkv;
        qkv.w = L.qkv;
        qkv.x = m->hidden;
        qkv.norm_gain = L.ln1;
        qkv.eps = c.rms_eps;
        qkv.bias = L.qkv_bias;
        qkv.y = m->qkv;
        CHIP_TRY(launch_gemv(qkv, s));
        // RoPE and the K/V append run inside the attention kernel where it
        // can (one launch fewer per layer), else as their own kernel.
        const bool fuse = attention_decode_fuses_rope(geom(m), (int)c.q_heads, (int)c.rotary_dim);
        if (!fuse)
            CHIP_TRY(launch_rope_append(m->qkv, m->qrot, 1, (int)c.q_heads, geom(m), L.kv, sh.rope_cos, sh.rope_sin,
                                        (int)c.rotary_dim, 0, pos, s));
        AttnJob aj;
        if (fuse) {
            aj.qkv = m->qkv;
            aj.rope_cos = sh.rope_cos;
            aj.rope_sin = sh.rope_sin;
            aj.rotary_dim = (int)c.rotary_dim;
        } else {
            aj.q = m->qrot;
        }
        aj.q_stride = sh.q_dim();
        aj.out = m->attn;
        aj.k = L.kv.k;
        aj.v = L.kv.v;
        aj.g = geom(m);
        aj.q_heads = (int)c.q_heads;
        aj.rows = 1;
        aj.pos_dev = pos;
        aj.splits = splits;
        aj.part = m->part;
        CHIP_TRY(launch_attention(aj, s));
        GemvJob o;
        o.w = L.o;
        o.x = m->attn;
        o.bias = L.o_bias;
        o.residual = m->hidden;
        o.epi = EPI_RESIDUAL;
        CHIP_TRY(launch_gemv(o, s));
        GemvJob gu;
        gu.w = L.gate;
        gu.w2 = L.up;
        gu.x = m->hidden;
        gu.norm_gain = L.ln2;
        gu.eps = c.rms_eps;
        gu.y = m->act;
        gu.epi = EPI_SWIGLU;
        CHIP_TRY(launch_gemv(gu, s));
        GemvJob dn;
        dn.w = L.down;
        dn.x = m->act;
        dn.residual = m->hidden;
        dn.epi = EPI_RESIDUAL;
        CHIP_TRY(launch_gemv(dn, s));
        CHIP_TRY(layer_end(m, l, s));
    }
    GemvJob head;
    head.w = sh.head;
    head.x = m->hidden;
    head.norm_gain = sh.final_norm;
    head.eps = c.rms_eps;
    head.y = m->logits;
    CHIP_TRY(launch_gemv(head, s));
    CHIP_TRY(launch_argmax(m->logits, c.vocab_size, m->next_dev, m->step_dev, m->hist_dev, sh.kv_capacity + 1,
                           m->argmax_scratch, s));
    return 0;
}

bool graphs_enabled() {
    const char *e = getenv("CHEETAH_HIP_GRAPH");
    return !(e && (e[0] == '0' || e[0] == 'f' || e[0] == 'F' || e[0] == 'n' || e[0] == 'N'));
}

// One decode step at absolute position `pos` (the device step word must
// already hold it): the captured graph for the step's split count.
int launch_decode(cheetah_hip_model *m, size_t pos) {
    const int splits = decode_splits(m, pos + 1);
    // Host-tier weights are fed by copies ordered with events on a second
    // stream: those steps run eagerly.
    if (!graphs_enabled() || m->sh->host_mats) return enqueue_decode(m, splits);
    if (splits < 1 || (size_t)splits >= m->graphs.size()) return fail("HIP backend: decode split count out of range.");
    hipGraphExec_t &exec = m->graphs[splits];
    if (!exec) {
        hipGraph_t g = nullptr;
        CHIP_CHECK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_decode(m, splits);
        hipError_t e = hipStreamEndCapture(m->stream, &g);
        if (rc != 0) {
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
        if (e != hipSuccess) return fail(std::string("HIP backend: decode graph capture failed: ") + hipGetErrorString(e));
        e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            exec = nullptr;
            return fail(std::string("HIP backend: decode graph instantiation failed: ") + hipGetErrorString(e));
        }
    }
    CHIP_CHECK(hipGraphLaunch(exec, m->stream));
    return 0;
}

int write_step(cheetah_hip_model *m, uint32_t token, size_t pos) {
    CHIP_CHECK(hipStreamSynchronize(m->stream));  // step_host may still be in flight
    m->step_host[0] = (int32_t)token;
    m->step_host[1] = (int32_t)pos;
    CHIP_CHECK(hipMemcpyAsync(m->step_dev, m->step_host, 2 * sizeof(int32_t), hipMemcpyHostToDevice, m->stream));
    return 0;
}

// One prefill chunk of `rows` tokens at absolute position `pos`.
// tokens_dev holds the chunk's ids (already on the device).
int enqueue_chunk(cheetah_hip_model *m, const uint32_t *tokens_dev, size_t rows, size_t pos, bool last_chunk) {
    Shared &sh = *m->sh;
    const auto &c = sh.cfg;
    hipStream_t s = m->stream;
    const size_t H = c.hidden_size;
    CHIP_TRY(launch_embed(sh.embed, H, tokens_dev, rows, m->hidden, s));
    // A fixed split count makes each row's split boundaries a function of its
    // own context length only, so a position's attention output does not
    // depend on how the prompt was cut into chunks (KV continuation stays
    // bit-exact, decoder.rs:1710-1728).
    const size_t splits = kPrefillSplits;
    // A residual GEMM that split K leaves its chunk sums in gemm_ws; the
    // reduction then runs fused with the RMSNorm that reads its output.
    int down_chunks = 0;
    const float *down_sc = nullptr;
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const Layer *Lp = nullptr;
        CHIP_TRY(layer_begin(m, l, s, &Lp));
        const Layer &L = *Lp;
        // The normed rows come with their BF16 halves (the GEMM's input).
        if (down_chunks)
            CHIP_TRY(launch_residual_rmsnorm_rows(m->gemm_ws, down_chunks, down_sc, nullptr, m->hidden, rows, H, L.ln1,
                                                  c.rms_eps, m->normed, s, m->xh, m->xl));
        else
            CHIP_TRY(launch_rmsnorm_rows(m->hidden, L.ln1, c.rms_eps, rows, H, m->normed, s, m->xh, m->xl));
        GemmJob qkv;
        qkv.w = L.qkv;
        qkv.x = m->normed;
        qkv.n = rows;
        qkv.bias = L.qkv_bias;
        qkv.y = m->qkv;
        qkv.ws = m->gemm_ws;
        qkv.ws_floats = m->gemm_ws_floats;
        qkv.xh = m->xh;
        qkv.xl = m->xl;
        // A split-K QKV GEMM leaves its chunk sums; the RoPE kernel folds them
        // (with the scale and bias) as it reads each element.
        int qkv_chunks = 0;
        qkv.deferred = &qkv_chunks;
        CHIP_TRY(launch_gemm(qkv, s));
        CHIP_TRY(launch_rope_append(m->qkv, m->qrot, rows, (int)c.q_heads, geom(m), L.kv, sh.rope_cos, sh.rope_sin,
                                    (int)c.rotary_dim, pos, nullptr, s, m->gemm_ws, qkv_chunks, L.qkv.scales(),
                                    L.qkv_bias));
        AttnJob aj;
        aj.q = m->qrot;
        aj.q_stride = sh.q_dim();
        aj.out = m->attn;
        aj.k = L.kv.k;
        aj.v = L.kv.v;
        aj.g = geom(m);
        aj.q_heads = (int)c.q_heads;
        aj.rows = rows;
        aj.offset = pos;
        aj.splits = (int)splits;
        aj.part = m->part;
        aj.part_floats = m->part_floats;
        aj.prefill = true;
        aj.span = attention_prefill_span(m->sh->kv_capacity);
        // The matrix-core prefill writes the o_proj input halves itself.
        const bool halves = attention_prefill_on_mfma(aj.g, aj.q_heads);
        if (halves) {
            aj.out_hi = m->xh;
            aj.out_lo = m->xl;
        }
        CHIP_TRY(launch_attention(aj, s));
        GemmJob o;
        o.w = L.o;
        o.x = m->attn;
        o.n = rows;
        o.bias = L.o_bias;
        o.residual = m->hidden;
        o.epi = EPI_RESIDUAL;
        o.ws = m->gemm_ws;
        o.ws_floats = m->gemm_ws_floats;
        if (!halves) CHIP_TRY(launch_split_bf16(m->attn, rows * (size_t)(sh.q_dim()), m->xh, m->xl, s));
        o.xh = m->xh;
        o.xl = m->xl;
        int o_chunks = 0;
        o.deferred = &o_chunks;
        CHIP_TRY(launch_gemm(o, s));
        if (o_chunks)
            CHIP_TRY(launch_residual_rmsnorm_rows(m->gemm_ws, o_chunks, L.o.scales(), L.o_bias, m->hidden, rows, H,
                                                  L.ln2, c.rms_eps, m->normed, s, m->xh, m->xl));
        else
            CHIP_TRY(launch_rmsnorm_rows(m->hidden, L.ln2, c.rms_eps, rows, H, m->normed, s, m->xh, m->xl));
        GemmJob gu;
        gu.w = L.gate;
        gu.w2 = L.up;
        gu.x = m->normed;
        gu.n = rows;
        gu.y = m->act;
        gu.epi = EPI_SWIGLU;
        gu.ws = m->gemm_ws;
        gu.ws_floats = m->gemm_ws_floats;
        gu.xh = m->xh;
        gu.xl = m->xl;
        gu.yh = m->ah;  // the down projection's input halves
        gu.yl = m->al;
        CHIP_TRY(launch_gemm(gu, s));
        GemmJob dn;
        dn.w = L.down;
        dn.x = m->act;
        dn.n = rows;
        dn.residual = m->hidden;
        dn.epi = EPI_RESIDUAL;
        dn.ws = m->gemm_ws;
        dn.ws_floats = m->gemm_ws_floats;
        dn.xh = m->ah;
        dn.xl = m->al;
        // A streamed layer's scales live in its feed slot, which is reused
        // once the layer ends: its reduction runs inside the layer (the same
        // chunk order, so the same bits).
        dn.deferred = L.streamed() ? nullptr : &down_chunks;
        down_chunks = 0;
        down_sc = L.down.scales();
        CHIP_TRY(launch_gemm(dn, s));
        CHIP_TRY(layer_end(m, l, s));
    }
    if (down_chunks)
        CHIP_TRY(launch_residual_rmsnorm_rows(m->gemm_ws, down_chunks, down_sc, nullptr, m->hidden, rows, H, nullptr,
                                              0.f, nullptr, s));
    if (last_chunk) {
        // Final norm of the last row only, fused into the LM head GEMV
        // (qwen2.rs:227-232 then lm_head, ops.rs:1513-1563).
        GemvJob head;
        head.w = sh.head;
        head.x = m->hidden + (rows - 1) * H;
        head.norm_gain = sh.final_norm;
        head.eps = c.rms_eps;
        head.y = m->logits;
        CHIP_TRY(launch_gemv(head, s));
    }
    return 0;
}

int check_model(const cheetah_hip_model *m) {
    if (!m) return fail("HIP backend: no model.");
    if (!m->sh->finalized) return fail("HIP backend: model not finalized; call cheetah_hip_model_finalize.");
    return ensure_ready();
}

// validate_tokens (ops.rs:1065-1078) + the device-backend offset contract
// (transformer.rs:799-810).
int validate(const cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset) {
    if (n == 0) return fail("HIP backend: empty token input.");
    if (!tokens) return fail("HIP backend: null token pointer.");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= C(m).vocab_size)
            return fail("HIP backend: token id " + std::to_string(tokens[i]) + " exceeds the vocabulary size " +
                        std::to_string(C(m).vocab_size) + ".");
    if (offset != m->len) return fail("HIP backend: KV cache position does not match the input offset.");
    if (offset + n > m->sh->kv_capacity)
        return fail("HIP backend: input exceeds the KV cache capacity of " + std::to_string(m->sh->kv_capacity) +
                    " positions.");
    return 0;
}

int validate_decode(const cheetah_hip_model *m, uint32_t token, size_t offset, size_t steps) {
    CHIP_TRY(validate(m, &token, 1, offset));
    if (offset + steps > m->sh->kv_capacity)
        return fail("HIP backend: decode exceeds the KV cache capacity of " + std::to_string(m->sh->kv_capacity) +
                    " positions.");
    return 0;
}

// Runs the forward; leaves the final logits in m->logits (and, for decode,
// the argmax in m->next_dev).
int run_forward(cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset, size_t chunk_rows) {
    CHIP_TRY(check_model(m));
    CHIP_TRY(validate(m, tokens, n, offset));
    CHIP_TRY(refresh_weights(m));
    if (chunk_rows == 0) chunk_rows = 256;
    chunk_rows = std::min(chunk_rows, m->sh->max_chunk);
    CHIP_TRY(reserve_positions(m, n));
    if (n == 1) {
        CHIP_TRY(write_step(m, tokens[0], offset));
        if (fused_fits(m, offset, 1)) CHIP_TRY(run_fused(m, offset, 1));
        else CHIP_TRY(launch_decode(m, offset));
    } else {
        CHIP_CHECK(hipStreamSynchronize(m->stream));  // tokens_host reuse
        std::memcpy(m->tokens_host, tokens, n * sizeof(uint32_t));
        CHIP_CHECK(hipMemcpyAsync(m->tokens_dev, m->tokens_host, n * sizeof(uint32_t), hipMemcpyHostToDevice,
                                  m->stream));
        for (size_t start = 0; start < n; start += chunk_rows) {
            const size_t rows = std::min(chunk_rows, n - start);
            CHIP_TRY(enqueue_chunk(m, m->tokens_dev + start, rows, offset + start, start + rows == n));
        }
        CHIP_TRY(launch_argmax(m->logits, C(m).vocab_size, m->next_dev, nullptr, nullptr, 0, m->argmax_scratch,
                               m->stream));
    }
    m->len = offset + n;
    return 0;
}

// A per-layer linear weight's unit id -> (layer, matrix index of
// Layer::mat); q, k and v all name the fused qkv matrix. False for every
// other id (embedding, norms, biases, head, unknown names).
bool parse_layer_unit(const Shared &sh, const char *id, uint32_t *layer, int *mat) {
    static const char *const names[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                        "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                                        "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                        "mlp.down_proj.weight"};
    static const int index[] = {0, 0, 0, 1, 2, 3, 4};
    const std::string s(id), prefix = "model.layers.";
    if (s.compare(0, prefix.size(), prefix) != 0) return false;
    size_t end = prefix.size();
    while (end < s.size() && s[end] >= '0' && s[end] <= '9') ++end;
    const size_t digits = end - prefix.size();
    if (digits == 0 || digits > 9 || end >= s.size() || s[end] != '.') return false;
    if (digits > 1 && s[prefix.size()] == '0') return false;
    const unsigned long l = std::stoul(s.substr(prefix.size(), digits));
    if (l >= sh.cfg.num_layers) return false;
    const std::string rest = s.substr(end + 1);
    for (int i = 0; i < 7; ++i)
        if (rest == names[i]) {
            *layer = (uint32_t)l;
            *mat = index[i];
            return true;
        }
    return false;
}

int read_logits(cheetah_hip_model *m, float *logits_out) {
    const size_t V = C(m).vocab_size;
    CHIP_CHECK(hipMemcpyAsync(m->logits_host, m->logits, V * sizeof(float), hipMemcpyDeviceToHost, m->stream));
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    std::memcpy(logits_out, m->logits_host, V * sizeof(float));
    return 0;
}

}  // namespace

extern "C" {

cheetah_hip_model *cheetah_hip_model_create(const cheetah_hip_config *cfg, uint32_t quant_format, uint32_t kv_format,
                                            size_t kv_capacity, size_t max_chunk_rows) {
    if (ensure_ready()) return nullptr;
    if (!cfg) {
        fail("HIP backend: null config.");
        return nullptr;
    }
    cheetah_hip_config c = *cfg;
    if (c.rotary_dim == 0) c.rotary_dim = c.head_dim;
    if (c.num_layers == 0 || c.hidden_size == 0 || c.q_heads == 0 || c.kv_heads == 0 || c.head_dim == 0 ||
        c.intermediate_size == 0 || c.vocab_size == 0 || c.q_heads % c.kv_heads != 0) {
        fail("HIP backend: invalid decoder configuration.");
        return nullptr;
    }
    if (c.family > 1) {
        fail("HIP backend: only the qwen2 (0) and llama (1) families are served.");
        return nullptr;
    }
    if (c.sliding_window != 0) {
        fail("HIP backend: sliding-window attention is not served (qwen2 and llama resolve it to 0).");
        return nullptr;
    }
    if ((c.head_dim != 64 && c.head_dim != 128) || c.q_heads / c.kv_heads > 8 || c.rotary_dim % 2 ||
        c.rotary_dim > c.head_dim) {
        fail("HIP backend: head_dim must be 64 or 128 with at most 8 query heads per KV head.");
        return nullptr;
    }
    if (c.hidden_size > 16384 || c.q_heads * c.head_dim > 16384 || c.intermediate_size > 32768) {
        fail("HIP backend: hidden / intermediate width above the served maximum.");
        return nullptr;
    }
    if (quant_format != 0 && quant_format != FMT_Q8 && quant_format != FMT_Q4) {
        fail("HIP backend: quant_format must be 0 (stored), 4 (q8) or 5 (q4).");
        return nullptr;
    }
    if (kv_format > 1) {
        fail("HIP backend: kv_format must be 0 (BF16) or 1 (f32).");
        return nullptr;
    }
    auto *m = new cheetah_hip_model();
    m->sh = std::make_shared<Shared>();
    m->sh->cfg = c;
    m->sh->quant = (int)quant_format;
    m->sh->kv_f32 = (int)kv_format;
    m->sh->kv_capacity = kv_capacity ? kv_capacity : 65536;
    m->sh->max_chunk = max_chunk_rows ? max_chunk_rows : 1024;
    return m;
}

int cheetah_hip_model_set_unit(cheetah_hip_model *m, const char *unit_id, const void *bytes, size_t nbytes,
                               uint32_t dtype, const uint64_t *shape, size_t ndim) {
    CHIP_TRY(ensure_ready());
    if (!m || !unit_id || !bytes || (ndim && !shape)) return fail("HIP backend: set_unit with a null argument.");
    if (m->sh->finalized) return fail("HIP backend: units cannot change after finalize.");
    if (dtype != 1) return fail(std::string("HIP backend: unit '") + unit_id + "' is not BF16 (the served stored precision).");
    if (ndim < 1 || ndim > 2) return fail(std::string("HIP backend: unit '") + unit_id + "' must be 1-D or 2-D.");
    uint64_t count = 1;
    for (size_t i = 0; i < ndim; ++i) count *= shape[i];
    if (count * 2 != nbytes)
        return fail(std::string("HIP backend: unit '") + unit_id + "' byte length does not match its shape.");
    Staged st;
    st.shape.assign(shape, shape + ndim);
    if (ndim == 2) {
        CHIP_CHECK(hipMalloc(&st.dev, nbytes));
        CHIP_CHECK(hipMemcpy(st.dev, bytes, nbytes, hipMemcpyHostToDevice));
    } else {
        st.host.resize(count);
        std::memcpy(st.host.data(), bytes, nbytes);
    }
    auto it = m->sh->staged.find(unit_id);
    if (it != m->sh->staged.end() && it->second.dev) (void)hipFree(it->second.dev);
    m->sh->staged[unit_id] = std::move(st);
    return 0;
}

int cheetah_hip_model_finalize(cheetah_hip_model *m) {
    CHIP_TRY(ensure_ready());
    if (!m) return fail("HIP backend: no model.");
    if (m->sh->finalized) return 0;
    CHIP_TRY(finalize(m));
    return init_instance(m);
}

int cheetah_hip_forward(cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset, size_t chunk_rows,
                        float *logits_out) {
    if (!logits_out) return fail("HIP backend: null logits buffer.");
    if (run_forward(m, tokens, n, offset, chunk_rows)) return -1;
    return read_logits(m, logits_out);
}

int cheetah_hip_forward_greedy(cheetah_hip_model *m, const uint32_t *tokens, size_t n, size_t offset,
                               size_t chunk_rows, uint32_t *next_token, float *logits_out) {
    if (!next_token) return fail("HIP backend: null next_token pointer.");
    if (run_forward(m, tokens, n, offset, chunk_rows)) return -1;
    CHIP_CHECK(hipMemcpyAsync(m->step_host, m->next_dev, sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    *next_token = (uint32_t)m->step_host[0];
    if (logits_out) CHIP_TRY(read_logits(m, logits_out));
    return 0;
}

int cheetah_hip_decode_greedy(cheetah_hip_model *m, uint32_t token, size_t offset, size_t steps,
                              uint32_t *tokens_out) {
    CHIP_TRY(check_model(m));
    if (steps == 0) return 0;
    if (!tokens_out) return fail("HIP backend: null tokens_out.");
    CHIP_TRY(validate_decode(m, token, offset, steps));
    CHIP_TRY(refresh_weights(m));
    CHIP_TRY(reserve_positions(m, steps));
    CHIP_TRY(write_step(m, token, offset));
    if (fused_fits(m, offset, steps)) CHIP_TRY(run_fused(m, offset, steps));
    else
        for (size_t i = 0; i < steps; ++i) CHIP_TRY(launch_decode(m, offset + i));
    CHIP_CHECK(hipMemcpyAsync(tokens_out, m->hist_dev + offset + 1, steps * sizeof(uint32_t), hipMemcpyDeviceToHost,
                              m->stream));
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    m->len = offset + steps;
    return 0;
}

int cheetah_hip_time_decode(cheetah_hip_model *m, uint32_t token, size_t offset, size_t steps, float *ms_per_step,
                            float *gemv_ms, uint32_t *tokens_out) {
    CHIP_TRY(check_model(m));
    if (steps == 0 || !ms_per_step) return fail("HIP backend: time_decode needs steps and an output.");
    CHIP_TRY(validate_decode(m, token, offset, steps));
    CHIP_TRY(refresh_weights(m));
    CHIP_TRY(reserve_positions(m, steps));
    CHIP_TRY(write_step(m, token, offset));
    hipEvent_t e0, e1;
    CHIP_CHECK(hipEventCreate(&e0));
    CHIP_CHECK(hipEventCreate(&e1));
    CHIP_CHECK(hipEventRecord(e0, m->stream));
    if (fused_fits(m, offset, steps)) {
        CHIP_TRY(run_fused(m, offset, steps));  // waits for the launch
    } else {
        for (size_t i = 0; i < steps; ++i) CHIP_TRY(launch_decode(m, offset + i));
    }
    CHIP_CHECK(hipEventRecord(e1, m->stream));
    CHIP_CHECK(hipEventSynchronize(e1));
    float total = 0.f;
    CHIP_CHECK(hipEventElapsedTime(&total, e0, e1));
    *ms_per_step = total / (float)steps;
    if (tokens_out)
        CHIP_CHECK(hipMemcpy(tokens_out, m->hist_dev + offset + 1, steps * sizeof(uint32_t), hipMemcpyDeviceToHost));
    m->len = offset + steps;
    if (gemv_ms && m->sh->host_mats) *gemv_ms = 0.f;  // the kernel alone needs every layer in HBM
    if (gemv_ms && !m->sh->host_mats) {
        // The dominant GEMV of the step (gate/up, SwiGLU epilogue, fused norm)
        // timed alone on the same stream, cycling through the layers so each
        // launch streams weights that are not cache resident.
        Shared &sh = *m->sh;
        const uint32_t L = sh.cfg.num_layers;
        const size_t iters = std::max<size_t>(steps, L);
        CHIP_CHECK(hipEventRecord(e0, m->stream));
        for (size_t i = 0; i < iters; ++i) {
            Layer &Ly = sh.layers[i % L];
            GemvJob gu;
            gu.w = Ly.gate;
            gu.w2 = Ly.up;
            gu.x = m->hidden;
            gu.norm_gain = Ly.ln2;
            gu.eps = sh.cfg.rms_eps;
            gu.y = m->act;
            gu.epi = EPI_SWIGLU;
            CHIP_TRY(launch_gemv(gu, m->stream));
        }
        CHIP_CHECK(hipEventRecord(e1, m->stream));
        CHIP_CHECK(hipEventSynchronize(e1));
        CHIP_CHECK(hipEventElapsedTime(&total, e0, e1));
        *gemv_ms = total / (float)iters;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

int cheetah_hip_evict_unit(cheetah_hip_model *m, const char *unit_id) {
    CHIP_TRY(check_model(m));
    if (!unit_id) return fail("HIP backend: null unit id.");
    Shared &sh = *m->sh;
    uint32_t l = 0;
    int i = 0;
    if (!parse_layer_unit(sh, unit_id, &l, &i)) return 0;
    Layer &L = sh.layers[l];
    if (L.host[i]) return 1;
    WMat &w = L.mat(i);
    // No kernel of any instance sharing these weights may still read them.
    CHIP_CHECK(hipDeviceSynchronize());
    uint8_t *h = nullptr;
    CHIP_CHECK(hipHostMalloc((void **)&h, w.bytes(), hipHostMallocDefault));
    const hipError_t e = hipMemcpy(h, w.base, w.bytes(), hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        (void)hipHostFree(h);
        return fail(std::string("HIP backend: evict copy failed: ") + hipGetErrorString(e));
    }
    sh.mem.release((void *)w.base);
    w.base = nullptr;
    L.host[i] = h;
    if (i == kLayerMats - 1 && L.down_cols) {
        // The persistent kernel's copy of this down_proj goes too (it is
        // rebuilt from the resident matrices once every unit is back).
        std::lock_guard<std::mutex> lock(sh.mu);
        sh.mem.release(L.down_cols);
        L.down_cols = nullptr;
        sh.down_cols_gen = 0;
    }
    ++sh.host_mats;
    ++sh.epoch;
    return 1;
}

int cheetah_hip_page_in_unit(cheetah_hip_model *m, const char *unit_id, int32_t tier) {
    (void)tier;  // every page-in lands in HBM
    CHIP_TRY(check_model(m));
    if (!unit_id) return fail("HIP backend: null unit id.");
    Shared &sh = *m->sh;
    uint32_t l = 0;
    int i = 0;
    if (!parse_layer_unit(sh, unit_id, &l, &i)) return 0;
    Layer &L = sh.layers[l];
    if (!L.host[i]) return 1;
    WMat &w = L.mat(i);
    // No feed copy may still read the host copy.
    CHIP_CHECK(hipDeviceSynchronize());
    uint8_t *d = nullptr;
    CHIP_TRY(sh.mem.alloc(&d, w.bytes()));
    const hipError_t e = hipMemcpy(d, L.host[i], w.bytes(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        sh.mem.release(d);
        return fail(std::string("HIP backend: page-in copy failed: ") + hipGetErrorString(e));
    }
    (void)hipHostFree(L.host[i]);
    L.host[i] = nullptr;
    w.base = d;
    --sh.host_mats;
    ++sh.epoch;
    return 1;
}

int cheetah_hip_unit_tier(const cheetah_hip_model *m, const char *unit_id) {
    CHIP_TRY(check_model(m));
    if (!unit_id) return fail("HIP backend: null unit id.");
    uint32_t l = 0;
    int i = 0;
    if (!parse_layer_unit(*m->sh, unit_id, &l, &i)) return 0;
    return m->sh->layers[l].host[i] ? 2 : 1;
}

void cheetah_hip_clear_cache(cheetah_hip_model *m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (int p : m->pages) m->sh->page_unref(p);
    m->pages.clear();
    m->len = 0;
}

cheetah_hip_model *cheetah_hip_clone(const cheetah_hip_model *src) {
    if (check_model(src)) return nullptr;
    auto *m = new cheetah_hip_model();
    m->sh = src->sh;
    if (init_instance(m)) {
        delete m;
        return nullptr;
    }
    return m;
}

size_t cheetah_hip_kv_len(const cheetah_hip_model *m) { return m ? m->len : 0; }

int cheetah_hip_kv_snapshot(const cheetah_hip_model *m, cheetah_hip_snapshot **out, size_t *positions) {
    CHIP_TRY(check_model(m));
    if (!out) return fail("HIP backend: null snapshot pointer.");
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    auto *s = new cheetah_hip_snapshot();
    s->sh = m->sh;
    s->positions = m->len;
    const size_t used = (m->len + kPageSize - 1) / kPageSize;
    for (size_t i = 0; i < used; ++i) {
        m->sh->page_ref(m->pages[i]);
        s->pages.push_back(m->pages[i]);
    }
    *out = s;
    if (positions) *positions = s->positions;
    return 0;
}

int cheetah_hip_restore_kv_prefix(cheetah_hip_model *m, const cheetah_hip_snapshot *s, size_t positions) {
    CHIP_TRY(check_model(m));
    if (!s) return fail("HIP backend: null snapshot.");
    if (s->sh != m->sh) return fail("HIP backend: snapshot belongs to another model's weights.");
    cheetah_hip_clear_cache(m);
    const size_t keep = std::min(positions, s->positions);
    const size_t used = (keep + kPageSize - 1) / kPageSize;
    for (size_t i = 0; i < used; ++i) {
        m->sh->page_ref(s->pages[i]);
        m->pages.push_back(s->pages[i]);
        m->page_host[i] = s->pages[i];
    }
    if (used) {
        CHIP_CHECK(hipMemcpyAsync(m->page_dev, m->page_host.data(), used * sizeof(int32_t), hipMemcpyHostToDevice,
                                  m->stream));
        CHIP_CHECK(hipStreamSynchronize(m->stream));
    }
    m->len = keep;
    return 0;
}

int cheetah_hip_kv_download(const cheetah_hip_model *m, uint32_t layer, size_t pos_begin, size_t n, float *k_out,
                            float *v_out) {
    CHIP_TRY(check_model(m));
    const Shared &sh = *m->sh;
    const cheetah_hip_config &c = sh.cfg;
    if (layer >= c.num_layers) return fail("HIP backend: kv_download layer out of range.");
    if (pos_begin > m->len || n > m->len - pos_begin)
        return fail("HIP backend: kv_download range exceeds the cached length " + std::to_string(m->len) + ".");
    if (n == 0) return 0;
    if (!k_out || !v_out) return fail("HIP backend: kv_download with a null output.");
    CHIP_CHECK(hipStreamSynchronize(m->stream));
    const size_t hd = c.head_dim, kvh = c.kv_heads, eb = sh.kv_f32 ? 4 : 2;
    const size_t pb = sh.page_bytes();
    std::vector<uint8_t> page(pb);
    const KvLayer &kv = sh.layers[layer].kv;
    for (int which = 0; which < 2; ++which) {
        const uint8_t *pool = (const uint8_t *)(which ? kv.v : kv.k);
        float *out = which ? v_out : k_out;
        for (size_t lp = pos_begin / kPageSize; lp <= (pos_begin + n - 1) / kPageSize; ++lp) {
            CHIP_CHECK(hipMemcpy(page.data(), pool + (size_t)m->pages[lp] * pb, pb, hipMemcpyDeviceToHost));
            const size_t p0 = std::max(pos_begin, lp * kPageSize);
            const size_t p1 = std::min(pos_begin + n, (lp + 1) * kPageSize);
            for (size_t p = p0; p < p1; ++p)
                for (size_t h = 0; h < kvh; ++h) {
                    const uint8_t *src = page.data() + ((h * kPageSize + p % kPageSize) * hd) * eb;
                    float *dst = out + ((p - pos_begin) * kvh + h) * hd;
                    for (size_t d = 0; d < hd; ++d) {
                        uint32_t bits;
                        if (eb == 4) {
                            std::memcpy(&bits, src + d * 4, 4);
                        } else {
                            uint16_t b16;
                            std::memcpy(&b16, src + d * 2, 2);
                            bits = (uint32_t)b16 << 16;  // BF16 widening is exact
                        }
                        std::memcpy(dst + d, &bits, 4);
                    }
                }
        }
    }
    return 0;
}

void cheetah_hip_snapshot_free(cheetah_hip_snapshot *s) { delete s; }

void cheetah_hip_model_free(cheetah_hip_model *m) { delete m; }

}  // extern "C"
