"""Parity of the isolated ops at the benchmark configurations, and of two
device behaviours the forward tests only reach through logits.

* Config 2: GQA attention 32 q / 8 KV heads, head_dim 128, BF16 K/V whose
  values are N(0, 1) rotated by RoPE (theta 1e6) at their positions: decode at
  1K / 4K / 16K keys and the 512-row causal chunk on a 4K cached prefix,
  against the oracle's attention_head (ops.rs:1357-1467).
* Config 3: Q8 and Q4 weight GEMM at N = 512 on 4096x4096, 4096x14336 and
  14336x4096, against the oracle's per-token gemv_q8 / gemv_q4
  (ops.rs:544-630) on a subsample of the 512 rows.
* Greedy ties: duplicated tied-embedding rows give bit-identical logits;
  every device argmax (prefill, captured-graph decode, persistent decode)
  must pick the last maximal index, as max_by(total_cmp) does
  (engine.rs:2247-2253).
* RoPE: with the K/V projection weights zeroed, the cached K rows are the
  rotated biases; they must equal the oracle's rope_heads (ops.rs:693-740)
  bit for bit (f32 cache) or after the BF16 rounding (BF16 cache).
"""
import numpy as np
import pytest

from cheetah_amd import configs, synth

pytestmark = pytest.mark.gpu

REL_BAR = 1e-2


@pytest.fixture(scope="module")
def hip():
    from cheetah_amd import hip as h
    h.init(0)
    return h


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _roped(oracle, x, heads, hd, positions, theta=1e6):
    """Rows x[i] (heads*hd) rotated at positions[i] by the oracle's rope."""
    return np.stack([oracle.rope_heads(x[i], heads, hd, hd, int(p), theta) for i, p in enumerate(positions)])


def _config2_cache(oracle, rng, ctx, kvh=8, hd=128):
    k = rng.standard_normal((ctx, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((ctx, kvh, hd)).astype(np.float32)
    k = _roped(oracle, k, kvh, hd, range(ctx)).reshape(ctx, kvh, hd)
    return synth.f32_to_bf16(k), synth.f32_to_bf16(v)


@pytest.mark.parametrize("ctx", [1024, 4096, 16384])
def test_config2_attention_decode(hip, oracle, ctx):
    q_heads, kvh, hd = 32, 8, 128
    rng = np.random.default_rng(ctx)
    kb, vb = _config2_cache(oracle, rng, ctx)
    q = rng.standard_normal((1, q_heads * hd)).astype(np.float32)
    q = synth.bf16_to_f32(synth.f32_to_bf16(_roped(oracle, q, q_heads, hd, [ctx - 1])))
    kp, vp, table = hip.paged_kv(kb, vb, seed=ctx)
    got = hip.attention(q, kp, vp, table, q_heads, 1, ctx - 1)[0]
    ref = oracle.attention(synth.bf16_to_f32(kb), synth.bf16_to_f32(vb), q[0], q_heads, kvh, hd, ctx - 1)
    assert np.max(np.abs(got - ref)) < 1e-4
    assert rel_err(got, ref) < REL_BAR


def test_config2_prefill_chunk_on_4k_prefix(hip, oracle):
    """512 query rows at positions 4096..4607, each attending causally to the
    cache (4096 cached positions plus the chunk's own rows)."""
    q_heads, kvh, hd, prefix, rows = 32, 8, 128, 4096, 512
    rng = np.random.default_rng(4608)
    kb, vb = _config2_cache(oracle, rng, prefix + rows)
    q = rng.standard_normal((rows, q_heads * hd)).astype(np.float32)
    q = synth.bf16_to_f32(synth.f32_to_bf16(_roped(oracle, q, q_heads, hd, range(prefix, prefix + rows))))
    kp, vp, table = hip.paged_kv(kb, vb, seed=7)
    got = hip.attention(q, kp, vp, table, q_heads, rows, prefix)
    kf, vf = synth.bf16_to_f32(kb), synth.bf16_to_f32(vb)
    for i in list(range(0, rows, 37)) + [rows - 1]:
        pos = prefix + i
        ref = oracle.attention(kf[: pos + 1], vf[: pos + 1], q[i], q_heads, kvh, hd, pos)
        assert np.max(np.abs(got[i] - ref)) < 1e-4, i


def _random_quant(rng, fmt, rows, cols):
    """Config-3 buffer: codes uniform over the full range, scales U[1e-3, 1e-2]."""
    scales = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)
    if fmt == "q8":
        stride = (cols + 3) // 4 * 4
        payload = np.zeros((rows, stride), np.uint8)
        payload[:, :cols] = rng.integers(-127, 128, (rows, cols)).astype(np.int8).view(np.uint8)
    else:
        stride = ((cols + 2) // 2 + 3) // 4 * 4
        nib = (rng.integers(-8, 8, (rows, cols)) & 0xF).astype(np.uint8)
        payload = np.zeros((rows, stride), np.uint8)
        payload[:, : (cols + 1) // 2] |= nib[:, 0::2]
        payload[:, : cols // 2] |= nib[:, 1::2] << 4
    return np.concatenate([scales.view(np.uint8), payload.reshape(-1)])


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (4096, 14336), (14336, 4096)])
def test_config3_quant_gemm_n512(hip, oracle, fmt, rows, cols):
    n = 512
    rng = np.random.default_rng(rows + cols + (5 if fmt == "q4" else 0))
    buf = _random_quant(rng, fmt, rows, cols)
    x = synth.bf16_to_f32(synth.f32_to_bf16(rng.standard_normal((n, cols)).astype(np.float32))).reshape(n, cols)
    got = hip.gemm(hip.DeviceBuffer.from_array(buf), fmt, rows, cols, x)
    sel = np.array(list(range(0, n, 37)) + [n - 1])
    ref = oracle.gemm_quant(buf, rows, cols, np.ascontiguousarray(x[sel]), fmt)
    assert rel_err(got[sel], ref) < 1e-4 < REL_BAR


# ---------------------------------------------------------------------------
# Greedy ties go to the last index.
# ---------------------------------------------------------------------------

def _oracle_greedy(oracle, shape, w, prompt, steps):
    r = oracle.RefModel(shape, w)
    logits = r.forward(prompt, 0, chunk_rows=16)
    toks, all_logits = [], []
    for s in range(steps):
        all_logits.append(logits)
        t = int(len(logits) - 1 - np.argmax(logits[::-1]))
        toks.append(t)
        if s + 1 < steps:
            logits = r.forward([t], len(prompt) + s)
    return toks, all_logits


def _with_row_copy(w, dst, src):
    w2 = dict(w)
    emb = w["model.embed_tokens.weight"].copy()
    emb[dst] = emb[src]
    w2["model.embed_tokens.weight"] = emb
    return w2


@pytest.mark.parametrize("step", [0, 1, 3])
@pytest.mark.parametrize("direction", ["above", "below"])
def test_greedy_ties_pick_the_last_index(hip, oracle, monkeypatch, step, direction):
    """The tied head of a tiny qwen2 gets a copy of the embedding row of the
    token greedy picks at `step`, at an index above or below it (another
    argmax block where one exists). The two logits are then bit-identical maxima; the oracle
    keeps the larger index, and so must the device's prefill argmax (step 0),
    graph decode and persistent decode (steps 1 and 3)."""
    shape = configs.TINY_QWEN2
    w = synth.make_weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 40, seed=12)
    base, _ = _oracle_greedy(oracle, shape, w, prompt, step + 1)
    b = base[step]
    used = set(prompt.tolist()) | set(base)
    cands = [j for j in range(shape.vocab_size) if j not in used and (j > b if direction == "above" else j < b)]
    if not cands:
        pytest.skip("no free index on that side of the greedy token")
    # Prefer another 512-index argmax block of the prefill argmax, then the
    # farthest index (another wave and block of the persistent head).
    j = min(cands, key=lambda c: ((c // 512) == (b // 512), -abs(c - b)))
    w2 = _with_row_copy(w, j, b)
    exp, exp_logits = _oracle_greedy(oracle, shape, w2, prompt, step + 3)
    lg = exp_logits[step]
    assert lg[j] == lg[b] == lg.max(), "the copied row must tie with the maximum"
    assert exp[step] == max(j, b)
    for mode in ("1", "0"):
        monkeypatch.setenv("CHEETAH_HIP_FUSED", mode)
        g = hip.HipForward(shape, w2, kv_capacity=512, max_chunk_rows=64)
        first, logits = g.forward_greedy(prompt, 0, chunk_rows=16, want_logits=True)
        rest = g.decode_greedy(first, len(prompt), step + 2)
        got = [first] + rest.tolist()
        assert got == exp, (mode, got, exp)
        if step == 0:
            assert logits[j].view(np.uint32) == logits[b].view(np.uint32)
        g.close()


# ---------------------------------------------------------------------------
# RoPE bit identity through the model's KV cache.
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_rope_of_cached_keys_is_bit_identical(hip, oracle, monkeypatch, kv):
    """k = 0 * x + bias exactly when k_proj is zero, so every cached K row is
    the bias rotated at its position (and every V row the bias): prefill
    chunks, graph decode and persistent decode must store the oracle's
    rope_heads bits (rounded to BF16 for the BF16 cache)."""
    shape = configs.TINY_QWEN2
    w = dict(synth.make_weights(shape))
    for layer in range(shape.num_layers):
        for n in ("k_proj", "v_proj"):
            key = f"model.layers.{layer}.self_attn.{n}.weight"
            w[key] = np.zeros_like(w[key])
    prompt = synth.make_tokens(shape.vocab_size, 70, seed=13)
    kvh, hd = shape.kv_heads, shape.head_dim
    for mode in ("1", "0"):
        monkeypatch.setenv("CHEETAH_HIP_FUSED", mode)
        g = hip.HipForward(shape, w, kv_capacity=512, max_chunk_rows=64, kv=kv)
        first = g.forward_greedy(prompt, 0, chunk_rows=32)
        g.decode_greedy(first, len(prompt), 12)
        n = g.kv_len()
        assert n == len(prompt) + 12
        for layer in range(shape.num_layers):
            p = f"model.layers.{layer}.self_attn."
            kb = synth.bf16_to_f32(w[p + "k_proj.bias"])
            vb = synth.bf16_to_f32(w[p + "v_proj.bias"])
            k_exp = np.stack([oracle.rope_heads(kb, kvh, hd, hd, pos, shape.rope_theta) for pos in range(n)])
            v_exp = np.broadcast_to(vb, (n, kvh * hd))
            if kv == "bf16":
                k_exp, v_exp = oracle.round_bf16(k_exp), oracle.round_bf16(np.ascontiguousarray(v_exp))
            k, v = g.kv_rows(layer, 0, n)
            assert np.array_equal(k.reshape(n, -1).view(np.uint32), k_exp.view(np.uint32)), (mode, layer)
            assert np.array_equal(v.reshape(n, -1).view(np.uint32),
                                  np.ascontiguousarray(v_exp, np.float32).view(np.uint32)), (mode, layer)
        g.close()
