"""Seeded random-init decoder weights and prompts.

Every tensor is drawn in blocks of 2^22 elements; block b of unit `name` comes
from ``numpy.random.Generator(PCG64(SeedSequence([seed, crc32(name), b])))``,
so any subset of units (or blocks) can be regenerated independently, blocks
are drawn in parallel, and the bytes are identical on every machine with the
same numpy. Linear weights and the embedding are normal(0, 0.02) in float32,
rounded to BF16 with round-to-nearest-even (the stored precision of a
prepared Cheetah model); RMSNorm gains are 1.0; qwen2 q/k/v biases are
normal(0, 0.02); there is no o_proj bias. Unit ids are the safetensors names
the reference's store serves (src/chat/native/store.rs:189-203).
"""
from __future__ import annotations

import os
import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .configs import DecoderShape

BF16_ONE = np.uint16(0x3F80)
BLOCK = 1 << 22


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """Round float32 to BF16 bits (round to nearest, ties to even; finite inputs)."""
    src = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(src.size, np.uint16)
    for s in range(0, src.size, BLOCK):
        bits = src[s:s + BLOCK].view(np.uint32)
        t = bits >> np.uint32(16)
        t &= np.uint32(1)
        t += np.uint32(0x7FFF)
        t += bits
        t >>= np.uint32(16)
        out[s:s + BLOCK] = t
    return out.reshape(np.shape(values))


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _block_values(seed: int, name: str, block: int, n: int, std: float) -> np.ndarray:
    ss = np.random.SeedSequence([seed, zlib.crc32(name.encode()), block])
    vals = np.random.Generator(np.random.PCG64(ss)).standard_normal(n, dtype=np.float32)
    vals *= np.float32(std)
    return f32_to_bf16(vals)


def unit_specs(shape: DecoderShape):
    """(unit id, tensor shape, kind) for every unit of the model."""
    specs = [("model.embed_tokens.weight", (shape.vocab_size, shape.hidden_size), "normal")]
    for layer in range(shape.num_layers):
        p = f"model.layers.{layer}."
        specs.append((p + "input_layernorm.weight", (shape.hidden_size,), "ones"))
        specs.append((p + "post_attention_layernorm.weight", (shape.hidden_size,), "ones"))
        for unit, rows, cols in shape.linear_units(layer):
            specs.append((unit, (rows, cols), "normal"))
        if shape.qkv_bias:
            specs.append((p + "self_attn.q_proj.bias", (shape.q_dim,), "normal"))
            specs.append((p + "self_attn.k_proj.bias", (shape.kv_dim,), "normal"))
            specs.append((p + "self_attn.v_proj.bias", (shape.kv_dim,), "normal"))
    specs.append(("model.norm.weight", (shape.hidden_size,), "ones"))
    if not shape.tie_word_embeddings:
        specs.append(("lm_head.weight", (shape.vocab_size, shape.hidden_size), "normal"))
    return specs


def _workers() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def make_weights(shape: DecoderShape, seed: int = 0, names=None, workers: int | None = None) -> dict:
    """Units as BF16 bit arrays (uint16), keyed by unit id (all, or `names`)."""
    specs = [s for s in unit_specs(shape) if names is None or s[0] in names]
    out = {}
    jobs = []
    for name, tshape, kind in specs:
        n = int(np.prod(tshape))
        if kind == "ones":
            out[name] = np.full(tshape, BF16_ONE, dtype=np.uint16)
            continue
        arr = np.empty(n, np.uint16)
        out[name] = arr.reshape(tshape)
        for b, s in enumerate(range(0, n, BLOCK)):
            jobs.append((arr, name, b, s, min(BLOCK, n - s)))

    def run(job):
        arr, name, b, s, cnt = job
        arr[s:s + cnt] = _block_values(seed, name, b, cnt, 0.02)

    with ThreadPoolExecutor(workers or _workers()) as ex:
        list(ex.map(run, jobs))
    return out


def make_tokens(vocab_size: int, count: int, seed: int = 1) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, vocab_size, size=count, dtype=np.uint32)
