"""The two large decoder workloads, driven through the HIP ModelForward the
way the reference's Engine drives a backend (engine.rs:1837-1979: clear,
optional prefix restore, chunked prompt forward, snapshot, greedy loop).

* Llama-3-8B shape, Q4 linears (quantized on the device from the seeded BF16
  weights, bit-exact to q4.rs:126-161), BF16 embedding/head/norms: an
  8192-token prompt in 512-row chunks, then greedy decode.
* Qwen2-7B shape, BF16 weights, BF16 (or f32) KV: turn 1 a 32768-token
  prompt in 1024-row chunks and a KV snapshot; turn 2 restores the first
  30720 positions, prefills a 2048-token suffix in 1024-row chunks, then
  decodes.

Each runner returns the sampled tokens and wall-clock phase timings
(synchronous forwards, so host time covers the device work).
"""
from __future__ import annotations

import time

import numpy as np

from . import configs, hip, synth


def greedy_token(logits) -> int:
    """Greedy sampling as the reference engine does it on the host: the
    index of the largest logit, the last one on ties (engine.rs:2247-2253).
    One forward argmax; the reversed search (a strided pass, about three
    times slower over a 152K vocabulary) runs only when a later logit ties
    the first maximum or the maximum is NaN."""
    logits = np.asarray(logits)
    i = int(np.argmax(logits))
    m = logits[i]
    if np.isnan(m) or (i + 1 < logits.size and logits[i + 1:].max() == m):
        return int(logits.size - 1 - np.argmax(logits[::-1]))
    return i


def _timed(fn, *args, **kw):
    t0 = time.perf_counter()
    out = fn(*args, **kw)
    hip.synchronize()
    return out, time.perf_counter() - t0


def load(shape, quant=None, kv: str = "bf16", kv_capacity: int = 0, max_chunk_rows: int = 0):
    t0 = time.perf_counter()
    weights = synth.make_weights(shape)
    t1 = time.perf_counter()
    g = hip.HipForward(shape, weights, quant=quant, kv=kv, kv_capacity=kv_capacity, max_chunk_rows=max_chunk_rows)
    del weights
    hip.synchronize()
    return g, {"synth_s": round(t1 - t0, 2), "upload_s": round(time.perf_counter() - t1, 2)}


def llama3_8b_q4(g=None, decode_steps: int = 256, prompt_len: int = 8192, chunk: int = 512, kv: str = "bf16"):
    shape = configs.LLAMA3_8B
    info = {}
    if g is None:
        g, info = load(shape, quant="q4", kv=kv, kv_capacity=prompt_len + decode_steps + 64, max_chunk_rows=chunk)
    prompt = synth.make_tokens(shape.vocab_size, prompt_len, seed=1)
    g.clear_cache()
    (first, logits), t_pre = _timed(g.forward_greedy, prompt, 0, chunk_rows=chunk, want_logits=True)
    rest, t_dec = _timed(g.decode_greedy, first, prompt_len, decode_steps - 1)
    tokens = [first] + rest.tolist()
    info.update({
        "prefill_s": round(t_pre, 4), "prefill_tok_s": round(prompt_len / t_pre, 1),
        "decode_s": round(t_dec, 4), "decode_tok_s": round((decode_steps - 1) / t_dec, 2),
        "tokens": tokens, "prefill_logits": logits,
    })
    return g, info


def qwen2_7b_32k(g=None, decode_steps: int = 128, prompt_len: int = 32768, reuse: int = 30720,
                 suffix_len: int = 2048, chunk: int = 1024, kv: str = "bf16"):
    shape = configs.QWEN2_7B
    info = {}
    if g is None:
        # The page pool holds the turn-1 snapshot (prompt_len positions) and
        # the pages turn 2 writes past the shared prefix.
        g, info = load(shape, kv=kv, kv_capacity=prompt_len + suffix_len + decode_steps + 64,
                       max_chunk_rows=chunk)
    prompt1 = synth.make_tokens(shape.vocab_size, prompt_len, seed=1)
    suffix = synth.make_tokens(shape.vocab_size, suffix_len, seed=2)
    g.clear_cache()
    (tok1, logits1), t_turn1 = _timed(g.forward_greedy, prompt1, 0, chunk_rows=chunk, want_logits=True)
    snap, t_snap = _timed(g.kv_snapshot)
    g.clear_cache()
    _, t_restore = _timed(g.restore_kv_prefix, snap, reuse)
    (first, logits2), t_turn2 = _timed(g.forward_greedy, suffix, reuse, chunk_rows=chunk, want_logits=True)
    rest, t_dec = _timed(g.decode_greedy, first, reuse + suffix_len, decode_steps - 1)
    del snap
    info.update({
        "turn1_prefill_s": round(t_turn1, 4), "turn1_prefill_tok_s": round(prompt_len / t_turn1, 1),
        "snapshot_s": round(t_snap, 4), "restore_s": round(t_restore, 4),
        "turn2_prefill_s": round(t_turn2, 4), "turn2_prefill_tok_s": round(suffix_len / t_turn2, 1),
        "decode_s": round(t_dec, 4), "decode_tok_s": round((decode_steps - 1) / t_dec, 2),
        "turn1_token": tok1, "turn1_logits": logits1, "turn2_logits": logits2,
        "tokens": [first] + rest.tolist(),
    })
    return g, info


def prefill_flops(shape, rows: int, offset: int = 0) -> float:
    """2 x linear params x rows + 4 * q_heads * head_dim * visible keys per
    layer (causal), the prefill FLOP count of a chunk run."""
    lin = 2.0 * shape.linear_params() * rows
    keys = rows * offset + rows * (rows + 1) / 2
    return lin + 4.0 * shape.q_heads * shape.head_dim * keys * shape.num_layers


def decode_bytes(shape, ctx: int, weight_bytes: float, kv_elem: int = 2) -> float:
    """Algorithmic bytes of one decode token at context ctx: every weight once
    (linears in their stored format, the BF16 head) + the K/V rows read, and
    one position written."""
    return weight_bytes + (ctx + 1) * shape.num_layers * 2 * shape.kv_dim * kv_elem
