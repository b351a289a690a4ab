"""Full-size decoder parity on the GPU against the oracle's golden runs.

Two KV precisions, two different claims:
* f32 KV cache: the reference's own semantics (ops.rs:995-999). The device
  must reproduce the reference's greedy tokens for the first 32 decode
  steps and its logits within 1e-2.
* BF16 KV cache (the served and timed default): a deliberate precision
  change. The device must reproduce the oracle run that rounds K/V to BF16
  on append; against the reference's tokens it may depart only at a step
  where the reference's own top-2 margin is a near-tie.

Every logit check covers the first 2048 logits and, where the golden holds
them, the whole vocabulary at 1/64 density plus the top 16, at the prefill
and at decode steps 1, 16 and 32.

Workloads:
* Llama-3-8B shape, Q4 linears, 8192-token prompt in 512-row chunks.
* Qwen2-7B shape, BF16, 32768-token prompt in 1024-row chunks, a KV snapshot,
  restore of the first 30720 positions, a 2048-token suffix, greedy decode.

The goldens come from tests/golden/make_golden.py (the oracle on this
container's CPU; hours of CPU time, so they are committed fixtures).
"""
import json
import os

import numpy as np
import pytest

import golden_checks

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


def _check_logits(got, head, sample=None):
    """First 2048 logits, and where the golden has them, every 64th logit of
    the whole vocabulary plus the golden's top 16, all within 1e-2."""
    got = np.asarray(got, np.float32)
    assert golden_checks.rel(got[: len(head)], head) < 1e-2
    if sample:
        golden_checks.check_vocab_sample(got, sample)


def _decode(g, first, position):
    """33 greedy tokens (the first from the prefill) with the logits of decode
    steps 1, 16 and 32 taken through the per-step forward."""
    return golden_checks.decode_sampled(g, first, position, 33)


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_llama3_8b_q4_8k_f32_kv_matches_reference(hip):
    gold = _load("llama3_8b_q4_greedy.json")
    assert gold["kv_cache"].startswith("f32")
    from cheetah_amd import workloads

    print("[large] llama3-8b q4, f32 KV, 8192-token prompt", flush=True)
    g, info = workloads.llama3_8b_q4(decode_steps=1, kv="f32")
    try:
        _check_logits(info["prefill_logits"], gold["prefill_logits_head"], gold.get("prefill_vocab_sample"))
        tokens, dec = _decode(g, info["tokens"][0], 8192)
        assert tokens[:32] == gold["tokens"][:32]
        golden_checks.check_decode_samples(dec, tokens, gold, required=True)
    finally:
        g.close()


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_llama3_8b_q4_8k_bf16_kv_32_greedy_steps(hip):
    """The device's BF16 KV cache against the oracle run that rounds K/V to
    BF16 on append: prefill logits within 1e-2 and the same 32 tokens.

    Against the reference (f32 KV) the BF16 cache misses both bars on this
    config, and the test states by how much: the prefill logits differ by
    ~2.5e-2 relative (8K positions of BF16-rounded K/V; the 1e-2 bar is met
    only by the f32 cache, test above), and the tokens may depart from the
    reference's only at a near-tie (reference top-2 margin below 0.05; 0.030
    at step 6 for this seed)."""
    gold = _load("llama3_8b_q4_bf16kv_greedy.json")
    ref = _load("llama3_8b_q4_greedy.json")
    from cheetah_amd import workloads

    print("[large] llama3-8b q4, bf16 KV, 8192-token prompt", flush=True)
    g, info = workloads.llama3_8b_q4(decode_steps=1, kv="bf16")
    try:
        _check_logits(info["prefill_logits"], gold["prefill_logits_head"], gold.get("prefill_vocab_sample"))
        tokens, dec = _decode(g, info["tokens"][0], 8192)
        assert tokens[:32] == gold["tokens"][:32]
        golden_checks.check_decode_samples(dec, tokens, gold, required=True)
        head = ref["prefill_logits_head"]
        vs_ref = golden_checks.rel(info["prefill_logits"][: len(head)], head)
        print(f"[large] bf16-KV prefill logits vs the reference: {vs_ref:.4f} relative", flush=True)
        assert vs_ref < 5e-2
        golden_checks.check_departure_at_near_tie(tokens, ref)
    finally:
        g.close()


def _qwen2_7b(hip, kv, gold):
    from cheetah_amd import workloads

    print(f"[large] qwen2-7b bf16 weights, {kv} KV, 32768-token prompt, restore 30720 + 2048", flush=True)
    g, info = workloads.qwen2_7b_32k(decode_steps=1, kv=kv)
    try:
        assert info["turn1_token"] == gold["turn1_token"]
        _check_logits(info["turn1_logits"], gold["turn1_logits_head"], gold.get("turn1_vocab_sample"))
        _check_logits(info["turn2_logits"], gold["turn2_logits_head"], gold.get("turn2_vocab_sample"))
        tokens, dec = _decode(g, info["tokens"][0], 32768)
        assert tokens[:32] == gold["tokens"][:32]
        # Both goldens hold whole-vocabulary samples of decode steps 1, 16
        # and 32 (tests/golden/make_golden.py).
        golden_checks.check_decode_samples(dec, tokens, gold, required=True)
    finally:
        g.close()
    return tokens


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_qwen2_7b_32k_f32_kv_matches_reference(hip):
    """Reference semantics (f32 KV) at 32K context: the turn-1 token, both
    turns' logits within 1e-2 and the first 32 decode ids equal the CPU
    path's."""
    gold = _load("qwen2_7b_32k_f32kv_greedy.json")
    assert gold["kv_cache"].startswith("f32")
    _qwen2_7b(hip, "f32", gold)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_qwen2_7b_32k_bf16_kv_32_greedy_steps(hip):
    """The BF16 cache against the oracle run with BF16 K/V. Against the
    reference-semantics (f32 KV) golden the device tokens may depart only at
    a near-tie (reference top-2 margin below 0.05; 0.0133 at step 10 for this
    seed): the measured cost of the BF16 cache at 32K context."""
    gold = _load("qwen2_7b_32k_greedy.json")
    tokens = _qwen2_7b(hip, "bf16", gold)
    ref = _load("qwen2_7b_32k_f32kv_greedy.json")
    assert gold["turn1_token"] == ref["turn1_token"]
    golden_checks.check_departure_at_near_tie(tokens, ref)
