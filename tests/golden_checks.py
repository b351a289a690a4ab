"""Shared checks of device runs against the oracle's golden fixtures.

A golden (tests/golden/make_golden.py) stores, besides the greedy ids and the
first 2048 prefill logits, whole-vocabulary samples: every 64th logit plus
the top 16 of the prefill logits and of the logits that pick the tokens of
decode steps 1, 16 and 32 (step k's logits come from the forward of token
k - 1 at position prompt + k - 1; step 0 is the prefill). The reference's
decoder tests compare whole logit vectors (decoder.rs:1440-1641); these
samples carry that check to the full-size configurations at 1/64 density.
"""
import numpy as np

DECODE_SAMPLE_STEPS = (1, 16, 32)


def rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def check_vocab_sample(got, sample, bar=1e-2, what="logits"):
    """Every 64th logit and the golden's top 16 within `bar` relative."""
    got = np.asarray(got, np.float32)
    e1 = rel(got[::64], sample["stride64"])
    top = np.array(sample["top16_ids"])
    e2 = rel(got[top], sample["top16_values"])
    assert e1 < bar and e2 < bar, f"{what}: stride-64 rel {e1:.3e}, top-16 rel {e2:.3e} (bar {bar})"
    return max(e1, e2)


def decode_sampled(g, first, position, steps, sample_steps=DECODE_SAMPLE_STEPS):
    """Greedy decode of `steps` tokens starting with `first` (token 0, at
    position `position`). The tokens of sample_steps come from the per-step
    forward with logits (ModelForward::forward's path); the runs between them
    from the device greedy loop. Returns (tokens, {step: logits})."""
    tokens, logits, k = [int(first)], {}, 1
    while k < steps:
        if k in sample_steps:
            tok, lg = g.forward_greedy([tokens[-1]], position + k - 1, want_logits=True)
            logits[k] = lg
            tokens.append(int(tok))
            k += 1
        else:
            nxt = min([s for s in sample_steps if s > k] + [steps])
            tokens += g.decode_greedy(tokens[-1], position + k - 1, nxt - k).tolist()
            k = nxt
    return tokens, logits


def check_decode_samples(logits, tokens, gold, bar=1e-2, required=True):
    """The sampled decode steps' logits against the golden's samples. A step
    is compared only while the device's tokens before it equal the golden's
    (after a departure the two runs see different inputs); the steps
    compared are returned with their errors."""
    samples = gold.get("decode_vocab_samples")
    if samples is None:
        assert not required, "golden has no decode_vocab_samples"
        return {}
    errs = {}
    for k, lg in sorted(logits.items()):
        if str(k) in samples and tokens[:k] == gold["tokens"][:k]:
            errs[k] = check_vocab_sample(lg, samples[str(k)], bar, what=f"decode step {k}")
    return errs


def first_departure(got, ref):
    return next((i for i in range(min(len(got), len(ref))) if got[i] != ref[i]), None)


def check_departure_at_near_tie(got, ref_gold, n=32, margin_bar=0.05):
    """BF16 K/V against the f32-KV reference: the tokens may depart, but only
    at a step where the reference's own top-2 margin is small (a near-tie
    that the K/V rounding can flip). Returns the step (None: no departure)."""
    first = first_departure(got[:n], ref_gold["tokens"][:n])
    if first is not None:
        m = ref_gold["top2_margins"][first]
        print(f"[golden] tokens depart from the reference at step {first}, reference top-2 margin {m:.4f}",
              flush=True)
        assert m < margin_bar, (first, m)
    return first
