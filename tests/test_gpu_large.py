"""Full-size decoder parity on the GPU against the oracle's golden runs.

* Llama-3-8B shape, Q4 linears, 8192-token prompt in 512-row chunks: the
  greedy ids of the first 32 decode steps equal the oracle's (the reference
  semantics: f32 KV cache), and the prefill logits agree within 1e-2; the
  same with the device's BF16 KV cache against the oracle run with BF16 K/V.
* Qwen2-7B shape, BF16, 32768-token prompt in 1024-row chunks, a KV snapshot,
  restore of the first 30720 positions, a 2048-token suffix and greedy decode:
  the same bars against the oracle run with a BF16 KV cache (the device's).

The goldens come from tests/golden/make_golden.py (the oracle on this
container's CPU; hours of CPU time, so they are committed fixtures).
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def hip():
    from cheetah_amd import hip as h
    h.init(0)
    return h


def _load(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f"golden {name} not generated")
    with open(path) as f:
        return json.load(f)


def _rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_llama3_8b_q4_8k_prefill_and_32_greedy_steps(hip):
    gold = _load("llama3_8b_q4_greedy.json")
    from cheetah_amd import workloads

    print("[large] llama3-8b q4, f32 KV, 8192-token prompt", flush=True)
    g, info = workloads.llama3_8b_q4(decode_steps=33, kv="f32")
    try:
        assert _rel(info["prefill_logits_head"], gold["prefill_logits_head"]) < 1e-2
        assert info["tokens"][:32] == gold["tokens"][:32]
    finally:
        g.close()


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_llama3_8b_q4_8k_bf16_kv_32_greedy_steps(hip):
    """The same workload with the device's BF16 KV cache, against the oracle
    run that rounds K/V to BF16 on append."""
    gold = _load("llama3_8b_q4_bf16kv_greedy.json")
    from cheetah_amd import workloads

    print("[large] llama3-8b q4, bf16 KV, 8192-token prompt", flush=True)
    g, info = workloads.llama3_8b_q4(decode_steps=33, kv="bf16")
    try:
        assert _rel(info["prefill_logits_head"], gold["prefill_logits_head"]) < 1e-2
        assert info["tokens"][:32] == gold["tokens"][:32]
    finally:
        g.close()


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_qwen2_7b_32k_prefill_prefix_reuse_and_32_greedy_steps(hip):
    gold = _load("qwen2_7b_32k_greedy.json")
    from cheetah_amd import workloads

    print("[large] qwen2-7b bf16, 32768-token prompt, restore 30720 + 2048", flush=True)
    g, info = workloads.qwen2_7b_32k(decode_steps=33)
    try:
        assert info["turn1_token"] == gold["turn1_token"]
        assert _rel(info["turn1_logits_head"], gold["turn1_logits_head"]) < 1e-2
        assert _rel(info["turn2_logits_head"], gold["turn2_logits_head"]) < 1e-2
        assert info["tokens"][:32] == gold["tokens"][:32]
    finally:
        g.close()
