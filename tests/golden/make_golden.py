"""Writes the greedy-decode golden fixtures from the CPU oracle.

Usage: python tests/golden/make_golden.py [qwen2_0_5b] [qwen2_0_5b_bf16kv]

Config 1: Qwen2-0.5B shape, seeded random-init BF16 weights (cheetah_amd.synth,
seed 0), 512 seeded prompt tokens (seed 1) prefilled in chunks of 128, then
greedy decode (argmax, ties to the last index, engine.rs:2247-2253) with the
reference's f32 KV cache. Stores the sampled ids, the top-2 margin of every
step, and the first 2048 prefill logits.
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


def make_qwen2_0_5b(steps=64, kv_bf16=False):
    shape = configs.QWEN2_0_5B
    w = synth.make_weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 512, seed=1)
    m = oracle.RefModel(shape, w, kv_bf16=kv_bf16)
    t0 = time.time()
    logits = m.forward(prompt, 0, chunk_rows=128)
    t_prefill = time.time() - t0
    head = logits[:2048].tolist()
    tokens, margins = [], []
    t0 = time.time()
    for step in range(steps):
        srt = np.sort(logits)
        margins.append(float(srt[-1] - srt[-2]))
        tok = greedy(logits)
        tokens.append(tok)
        if step + 1 < steps:
            logits = m.forward([tok], 512 + step)
    t_decode = time.time() - t0
    return {
        "config": "qwen2-0.5b bf16, weights seed 0, prompt seed 1",
        "kv_cache": "bf16 (K/V rounded to nearest even on append)" if kv_bf16 else "f32 (reference)",
        "prompt_len": 512, "prompt_seed": 1, "chunk_rows": 128,
        "tokens": tokens, "top2_margins": margins, "prefill_logits_head": head,
        "oracle_threads": oracle.get_threads(),
        "oracle_seconds": {"prefill": round(t_prefill, 3), "decode": round(t_decode, 3)},
    }


MAKERS = {
    "qwen2_0_5b": make_qwen2_0_5b,
    "qwen2_0_5b_bf16kv": lambda: make_qwen2_0_5b(kv_bf16=True),
}

if __name__ == "__main__":
    which = sys.argv[1:] or list(MAKERS)
    for name in which:
        data = MAKERS[name]()
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}_greedy.json")
        with open(path, "w") as f:
            json.dump(data, f)
        print(path, data["tokens"][:16], min(data["top2_margins"][:32]))
