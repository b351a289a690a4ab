"""Forward-level checks of the CPU oracle: the reference's bit-exact decoder
invariants (src/chat/native/decoder.rs:1710-1860) and an independent float64
tensor-math forward (the ref_mat / ref_rope pattern, decoder.rs:1367-1530).
"""
import math

import numpy as np
import pytest

from cheetah_amd import configs, synth


def _model(oracle, shape, quant=None, seed=0):
    w = synth.make_weights(shape, seed=seed)
    return oracle.RefModel(shape, w, quant=quant), w


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("shape", [configs.TINY_QWEN2, configs.TINY_LLAMA], ids=lambda s: s.name)
def test_chunked_prefill_equals_per_position(oracle, shape):
    # decoder.rs:1824-1860: 53 tokens, chunk 16 and 8, non-zero offset.
    m, _ = _model(oracle, shape)
    toks = synth.make_tokens(shape.vocab_size, 53, seed=3)
    ref = None
    for chunk in (1, 8, 16, 256):
        m.clear_cache()
        m.forward(toks[:5], 0, chunk_rows=chunk)
        out = m.forward(toks[5:], 5, chunk_rows=chunk)
        if ref is None:
            ref = out
        assert np.array_equal(_bits(out), _bits(ref)), chunk


def test_kv_continuation_and_snapshot_restore_bit_exact(oracle):
    # decoder.rs:1710-1728 (continuation) and 1795-1818 (snapshot restore).
    shape = configs.TINY_QWEN2
    m, _ = _model(oracle, shape)
    toks = synth.make_tokens(shape.vocab_size, 20, seed=4)
    full = m.forward(toks, 0)
    m.clear_cache()
    m.forward(toks[:12], 0)
    snap = m.kv_snapshot()
    assert snap.positions == 12
    cont = m.forward(toks[12:], 12)
    assert np.array_equal(_bits(full), _bits(cont))
    other = m.clone()
    assert other.kv_len() == 0  # decoder.rs:1761-1788: a clone starts empty
    assert other.restore_kv_prefix(snap, 10)
    assert other.kv_len() == 10
    again = other.forward(toks[10:], 10)
    assert np.array_equal(_bits(full), _bits(again))


def test_clear_cache_isolation(oracle):
    # decoder.rs:1733-1756.
    shape = configs.TINY_LLAMA
    m, _ = _model(oracle, shape)
    a = synth.make_tokens(shape.vocab_size, 9, seed=5)
    b = synth.make_tokens(shape.vocab_size, 9, seed=6)
    first = m.forward(a, 0)
    m.clear_cache()
    m.forward(b, 0)
    m.clear_cache()
    assert np.array_equal(_bits(m.forward(a, 0)), _bits(first))


def test_token_validation_errors(oracle):
    # ops.rs:1065-1078.
    shape = configs.TINY_QWEN2
    m, _ = _model(oracle, shape)
    with pytest.raises(ValueError, match="empty token input"):
        m.forward(np.array([], np.uint32), 0)
    with pytest.raises(ValueError, match="exceeds the vocabulary size 1000"):
        m.forward(np.array([1000], np.uint32), 0)


def rne_bf16(values) -> np.ndarray:
    """Round to the nearest BF16, ties to the even BF16, chosen by comparing
    float64 distances to the two BF16 neighbours of each f32 value (an
    independent statement of the rule: no bit-pattern carry trick)."""
    x = np.ascontiguousarray(values, np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    toward0 = (bits & 0xFFFF0000).astype(np.uint32)
    away = (toward0.astype(np.uint64) + 0x10000).astype(np.uint32)
    lo = toward0.view(np.float32).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        hi = away.view(np.float32).astype(np.float64)
        # Past the largest BF16 the upper neighbour is 2^128 (stored as inf).
        hi = np.where((away & 0x7FFFFFFF) == 0x7F800000, np.copysign(2.0 ** 128, x.astype(np.float64)), hi)
        d_lo = np.abs(x.astype(np.float64) - lo)
        d_hi = np.abs(hi - x.astype(np.float64))
    odd = ((toward0 >> 16) & 1) == 1
    pick_hi = (bits & 0xFFFF != 0) & ((d_hi < d_lo) | ((d_hi == d_lo) & odd))
    return np.where(pick_hi, away, toward0).view(np.float32)


def numpy_forward(shape, w, tokens, kv_bf16=False):
    """float64 tensor-math forward of the qwen2/llama block
    (decoder.rs:1367-1433 helper pattern); kv_bf16 rounds every cached K and
    V element (after RoPE) to BF16, as the BF16-KV cache stores it."""
    f = lambda name: synth.bf16_to_f32(w[name]).astype(np.float64)
    H, hd = shape.hidden_size, shape.head_dim
    n = len(tokens)
    x = f("model.embed_tokens.weight")[tokens]

    def rms(v, g):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + shape.rms_eps) * g

    half = hd // 2
    inv = shape.rope_theta ** (-2.0 * np.arange(half) / hd)
    ang = np.arange(n)[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(t, heads):
        t = t.reshape(n, heads, hd)
        a, b = t[..., :half], t[..., half:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([a * c - b * s, b * c + a * s], -1)

    G = shape.q_heads // shape.kv_heads
    mask = np.tril(np.ones((n, n), bool))
    for layer in range(shape.num_layers):
        p = f"model.layers.{layer}."
        hn = rms(x, f(p + "input_layernorm.weight"))
        q = hn @ f(p + "self_attn.q_proj.weight").T
        k = hn @ f(p + "self_attn.k_proj.weight").T
        v = hn @ f(p + "self_attn.v_proj.weight").T
        if shape.qkv_bias:
            q += f(p + "self_attn.q_proj.bias")
            k += f(p + "self_attn.k_proj.bias")
            v += f(p + "self_attn.v_proj.bias")
        q, k = rope(q, shape.q_heads), rope(k, shape.kv_heads)
        v = v.reshape(n, shape.kv_heads, hd)
        if kv_bf16:
            k = rne_bf16(k).astype(np.float64)
            v = rne_bf16(v).astype(np.float64)
        out = np.zeros((n, shape.q_heads, hd))
        for h in range(shape.q_heads):
            s = q[:, h] @ k[:, h // G].T / math.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            pr = np.exp(s - s.max(-1, keepdims=True))
            pr /= pr.sum(-1, keepdims=True)
            out[:, h] = pr @ v[:, h // G]
        x = x + out.reshape(n, -1) @ f(p + "self_attn.o_proj.weight").T
        hn = rms(x, f(p + "post_attention_layernorm.weight"))
        g = hn @ f(p + "mlp.gate_proj.weight").T
        u = hn @ f(p + "mlp.up_proj.weight").T
        x = x + (g / (1 + np.exp(-g)) * u) @ f(p + "mlp.down_proj.weight").T
    last = rms(x[-1], f("model.norm.weight"))
    head = "model.embed_tokens.weight" if shape.tie_word_embeddings else "lm_head.weight"
    return f(head) @ last


@pytest.mark.parametrize("shape", [configs.TINY_QWEN2, configs.TINY_LLAMA], ids=lambda s: s.name)
def test_forward_matches_float64_tensor_math(oracle, shape):
    m, w = _model(oracle, shape)
    toks = synth.make_tokens(shape.vocab_size, 11, seed=7)
    got = m.forward(toks, 0, chunk_rows=4)
    exp = numpy_forward(shape, w, toks)
    assert np.max(np.abs(got - exp)) < 1e-4 * max(1.0, np.max(np.abs(exp)))


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_quantized_forward_uses_quantize_then_gemv(oracle, fmt):
    # ops.rs:1199-1226: under CHEETAH_QUANT_Q* every linear computes from the
    # quantized buffer; the result equals a bf16 model whose linear weights
    # are replaced by their dequantized values, up to accumulation order.
    shape = configs.TINY_QWEN2
    w = synth.make_weights(shape)
    mq = oracle.RefModel(shape, w, quant=fmt)
    deq_w = dict(w)
    for layer in range(shape.num_layers):
        for unit, rows, cols in shape.linear_units(layer):
            buf = oracle.quantize(synth.bf16_to_f32(w[unit]).reshape(rows, cols), fmt)
            deq_w[unit] = oracle.dequant(buf, rows, cols, fmt)  # float32 units
    mf = oracle.RefModel(shape, deq_w)
    toks = synth.make_tokens(shape.vocab_size, 6, seed=8)
    a = mq.forward(toks, 0)
    b = mf.forward(toks, 0)
    assert np.max(np.abs(a - b)) < 1e-4 * max(1.0, np.max(np.abs(b)))


def test_round_bf16_matches_nearest_even(oracle):
    """The oracle's BF16-KV rounding (a bit-pattern carry) against the
    distance-based statement above, on hand-picked cases and on random bit
    patterns of every exponent."""
    eps8 = 2.0 ** -8  # half a BF16 ulp at 1.0
    cases = {
        1.0 + eps8: 1.0,                         # tie, even neighbour below
        1.0 + 3 * eps8: 1.0 + 4 * eps8,          # tie, even neighbour above
        1.0 + eps8 + 2.0 ** -20: 1.0 + 2 * eps8, # just past the tie
        -(1.0 + eps8): -1.0,
        -(1.0 + 3 * eps8): -(1.0 + 4 * eps8),
        65504.0: 65536.0,
        float(np.finfo(np.float32).max): np.inf,  # past the largest BF16
        -float(np.finfo(np.float32).max): -np.inf,
        2.0 ** -130: 2.0 ** -130,                # subnormal, exact in BF16
        0.0: 0.0,
    }
    src = np.array(list(cases), np.float32)
    got = oracle.round_bf16(src)
    assert np.array_equal(got, np.array(list(cases.values()), np.float32)), (src, got)
    assert oracle.round_bf16(np.array([-0.0], np.float32)).view(np.uint32)[0] == 0x80000000
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite values only
    x = bits.view(np.float32)
    assert np.array_equal(oracle.round_bf16(x).view(np.uint32), rne_bf16(x).view(np.uint32))
    # The rounding is idempotent and leaves BF16 values alone.
    r = oracle.round_bf16(x)
    assert np.array_equal(oracle.round_bf16(r).view(np.uint32), r.view(np.uint32))


@pytest.mark.parametrize("shape", [configs.TINY_QWEN2, configs.TINY_LLAMA], ids=lambda s: s.name)
def test_bf16_kv_forward_matches_float64_with_rounded_cache(oracle, shape):
    """The oracle's BF16-KV mode against the float64 forward whose cached K
    and V are rounded to BF16: agreement within 1e-5 of the largest logit
    (measured ~5e-7), while the same float64 forward without the rounding
    lies ~1e-3 away, so a dropped or partial (K-only) rounding fails here."""
    w = synth.make_weights(shape)
    m = oracle.RefModel(shape, w, kv_bf16=True)
    toks = synth.make_tokens(shape.vocab_size, 23, seed=9)
    got = m.forward(toks, 0, chunk_rows=8).astype(np.float64)
    exp = numpy_forward(shape, w, toks, kv_bf16=True)
    unrounded = numpy_forward(shape, w, toks, kv_bf16=False)
    scale = max(1.0, np.max(np.abs(exp)))
    err = np.max(np.abs(got - exp)) / scale
    err_unrounded = np.max(np.abs(got - unrounded)) / scale
    assert err < 1e-5, err
    assert err_unrounded > 100 * err, (err, err_unrounded)
