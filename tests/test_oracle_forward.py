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


def numpy_forward(shape, w, tokens):
    """float64 tensor-math forward of the qwen2/llama block
    (decoder.rs:1367-1433 helper pattern)."""
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
