"""Writes the greedy-decode golden fixtures from the CPU oracle.

Usage: python tests/golden/make_golden.py [name ...]   (names: the MAKERS keys)

Config 1: Qwen2-0.5B shape, seeded random-init BF16 weights (cheetah_amd.synth,
seed 0), 512 seeded prompt tokens (seed 1) prefilled in chunks of 128, then
greedy decode (argmax, ties to the last index, engine.rs:2247-2253) with the
reference's f32 KV cache. Stores the sampled ids, the top-2 margin of every
step, the first 2048 prefill logits, and whole-vocabulary samples (every 64th
logit plus the top 16) of the prefill logits and of the logits that pick the
tokens of decode steps 1, 16 and 32 (step k's logits come from the forward of
token k - 1; step 0 is the prefill).
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from cheetah_amd import configs, synth  # noqa: E402
from oracle import oracle  # noqa: E402


def greedy(logits):
    return int(len(logits) - 1 - np.argmax(logits[::-1]))


DECODE_SAMPLE_STEPS = (1, 16, 32)


def _vocab_sample(logits):
    """Every 64th logit plus the top 16 (index, value): a full-vocabulary check
    that stays a few KB."""
    top = np.argsort(logits)[::-1][:16]
    return {"stride64": logits[::64].tolist(), "top16_ids": top.tolist(),
            "top16_values": logits[top].tolist()}


def _decode(m, logits, position, steps):
    """Greedy decode from the prompt's logits: the ids, the top-2 margin of
    every step and the vocabulary samples at DECODE_SAMPLE_STEPS."""
    tokens, margins, samples = [], [], {}
    for step in range(steps):
        if step in DECODE_SAMPLE_STEPS:
            samples[str(step)] = _vocab_sample(logits)
        srt = np.sort(logits)
        margins.append(float(srt[-1] - srt[-2]))
        tok = greedy(logits)
        tokens.append(tok)
        if step + 1 < steps:
            logits = m.forward([tok], position + step)
    return tokens, margins, samples


def make_qwen2_0_5b(steps=64, kv_bf16=False):
    shape = configs.QWEN2_0_5B
    w = synth.make_weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 512, seed=1)
    m = oracle.RefModel(shape, w, kv_bf16=kv_bf16)
    t0 = time.time()
    logits = m.forward(prompt, 0, chunk_rows=128)
    t_prefill = time.time() - t0
    head = logits[:2048].tolist()
    prefill_sample = _vocab_sample(logits)
    t0 = time.time()
    tokens, margins, samples = _decode(m, logits, 512, steps)
    t_decode = time.time() - t0
    return {
        "config": "qwen2-0.5b bf16, weights seed 0, prompt seed 1",
        "kv_cache": "bf16 (K/V rounded to nearest even on append)" if kv_bf16 else "f32 (reference)",
        "prompt_len": 512, "prompt_seed": 1, "chunk_rows": 128,
        "tokens": tokens, "top2_margins": margins, "prefill_logits_head": head,
        "prefill_vocab_sample": prefill_sample, "decode_vocab_samples": samples,
        "oracle_threads": oracle.get_threads(),
        "oracle_seconds": {"prefill": round(t_prefill, 3), "decode": round(t_decode, 3)},
    }


def make_llama3_8b_q4(steps=40, kv_bf16=False):
    """Config 4: Llama-3-8B shape, Q4 linears quantized from the seeded BF16
    weights (q4.rs:126-161), BF16 embedding/head/norms; an 8192-token prompt
    (seed 1) in 512-row chunks, then greedy decode."""
    shape = configs.LLAMA3_8B
    w = synth.make_weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 8192, seed=1)
    m = oracle.RefModel(shape, w, quant="q4", kv_bf16=kv_bf16)
    t0 = time.time()
    logits = m.forward(prompt, 0, chunk_rows=512)
    t_prefill = time.time() - t0
    head = logits[:2048].tolist()
    prefill_sample = _vocab_sample(logits)
    t0 = time.time()
    tokens, margins, samples = _decode(m, logits, 8192, steps)
    return {
        "config": "llama3-8b q4 (linears), bf16 embedding/head/norms, weights seed 0, prompt seed 1",
        "kv_cache": "bf16 (K/V rounded to nearest even on append)" if kv_bf16 else "f32 (reference)",
        "prompt_len": 8192, "prompt_seed": 1, "chunk_rows": 512,
        "tokens": tokens, "top2_margins": margins, "prefill_logits_head": head,
        "prefill_vocab_sample": prefill_sample, "decode_vocab_samples": samples,
        "oracle_threads": oracle.get_threads(),
        "oracle_seconds": {"prefill": round(t_prefill, 3), "decode": round(time.time() - t0, 3)},
    }


def make_qwen2_7b_32k(steps=40, kv_bf16=True):
    """Config 5: Qwen2-7B shape, BF16 weights, BF16 KV (kv_bf16) or the
    reference's f32 KV (ops.rs:995-999). Turn 1: a
    32768-token prompt (seed 1) in 1024-row chunks, KV snapshot. Turn 2: the
    first 30720 prompt tokens + 2048 new ones (seed 2); the prefix is restored
    from the snapshot (engine.rs:523-601 semantics), the suffix prefilled in
    1024-row chunks, then greedy decode."""
    shape = configs.QWEN2_7B
    w = synth.make_weights(shape)
    prompt1 = synth.make_tokens(shape.vocab_size, 32768, seed=1)
    suffix = synth.make_tokens(shape.vocab_size, 2048, seed=2)
    m = oracle.RefModel(shape, w, kv_bf16=kv_bf16)
    del w
    t0 = time.time()
    logits1 = m.forward(prompt1, 0, chunk_rows=1024)
    t_turn1 = time.time() - t0
    snap = m.kv_snapshot()
    m.clear_cache()
    assert m.restore_kv_prefix(snap, 30720)
    del snap
    t0 = time.time()
    logits2 = m.forward(suffix, 30720, chunk_rows=1024)
    t_turn2 = time.time() - t0
    t0 = time.time()
    tokens, margins, samples = _decode(m, logits2, 32768, steps)
    srt = np.sort(logits1)
    return {
        "config": "qwen2-7b bf16, weights seed 0; turn 1 prompt seed 1 (32768), turn 2 = first 30720 + 2048 "
                  "tokens of seed 2",
        "kv_cache": "bf16 (K/V rounded to nearest even on append)" if kv_bf16 else "f32 (reference)",
        "prompt_len": 32768, "prefix_reused": 30720, "suffix_len": 2048, "suffix_seed": 2, "chunk_rows": 1024,
        "turn1_token": greedy(logits1), "turn1_margin": float(srt[-1] - srt[-2]),
        "turn1_logits_head": logits1[:2048].tolist(), "turn2_logits_head": logits2[:2048].tolist(),
        "turn1_vocab_sample": _vocab_sample(logits1), "turn2_vocab_sample": _vocab_sample(logits2),
        "tokens": tokens, "top2_margins": margins, "decode_vocab_samples": samples,
        "oracle_threads": oracle.get_threads(),
        "oracle_seconds": {"turn1_prefill": round(t_turn1, 3), "turn2_prefill": round(t_turn2, 3),
                           "decode": round(time.time() - t0, 3)},
    }


MAKERS = {
    "qwen2_0_5b": make_qwen2_0_5b,
    "qwen2_0_5b_bf16kv": lambda: make_qwen2_0_5b(kv_bf16=True),
    "llama3_8b_q4": make_llama3_8b_q4,
    "llama3_8b_q4_bf16kv": lambda: make_llama3_8b_q4(kv_bf16=True),
    "qwen2_7b_32k": make_qwen2_7b_32k,
    "qwen2_7b_32k_f32kv": lambda: make_qwen2_7b_32k(kv_bf16=False),
}

if __name__ == "__main__":
    if os.environ.get("CHEETAH_REF_THREADS"):
        oracle.set_threads(int(os.environ["CHEETAH_REF_THREADS"]))
    which = sys.argv[1:] or list(MAKERS)
    for name in which:
        data = MAKERS[name]()
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}_greedy.json")
        with open(path, "w") as f:
            json.dump(data, f)
        print(path, data["tokens"][:16], min(data["top2_margins"][:32]), data["oracle_seconds"], flush=True)
