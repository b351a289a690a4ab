"""Ant tier control on the device (AntTierControl::page_in_unit / evict_unit,
registry.rs:87-93, driven by engine.rs:1210-1226).

An evicted per-layer weight leaves HBM for pinned host memory and is streamed
into a device slot one layer ahead of the compute; the kernels that read it
are the same, so every logit must keep its bits. The decode comparisons run
the per-kernel path on both sides (CHEETAH_HIP_FUSED=0), since the persistent
kernel only runs while every layer is resident; after page-in the persistent
kernel is checked against a never-evicted model.
"""
import numpy as np
import pytest

from cheetah_amd import configs, synth

pytestmark = pytest.mark.gpu

_WEIGHTS = {}


@pytest.fixture(scope="module")
def hip():
    from cheetah_amd import hip as h
    h.init(0)
    return h


def weights(shape):
    if shape.name not in _WEIGHTS:
        _WEIGHTS.clear()
        _WEIGHTS[shape.name] = synth.make_weights(shape)
    return _WEIGHTS[shape.name]


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def unit(l, name):
    return f"model.layers.{l}.{name}.weight"


ALL = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
       "mlp.up_proj", "mlp.down_proj"]


def run(g, prompt, steps, chunk_rows):
    """Prefill logits + greedy tokens + the logits of one more decode step."""
    first, pre = g.forward_greedy(prompt, 0, chunk_rows=chunk_rows, want_logits=True)
    toks = g.decode_greedy(first, len(prompt), steps)
    last = g.forward(toks[-1:], len(prompt) + steps)
    return pre, [first] + toks.tolist(), last


# Evicted units per case: consecutive layers, same-parity layers with a
# resident one between, single matrices (k_proj moves the fused q/k/v), and
# the last layer (its prefetch wraps to the first streamed layer).
CASES = [
    (configs.QWEN2_0_5B, None, [(0, ALL), (1, ["mlp.down_proj"]), (5, ["self_attn.k_proj", "mlp.up_proj"]),
                                (7, ["self_attn.o_proj"]), (23, ALL)]),
    (configs.TINY_LLAMA, "q4", [(1, ["mlp.down_proj", "mlp.gate_proj"])]),
    (configs.TINY_QWEN2, "q8", [(0, ALL), (1, ALL)]),
]


@pytest.mark.parametrize("shape,quant,evict", CASES, ids=lambda c: getattr(c, "name", None))
def test_evicted_units_stream_bit_identical(hip, shape, quant, evict, monkeypatch):
    monkeypatch.setenv("CHEETAH_HIP_FUSED", "0")
    w = weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 150, seed=21)
    kw = dict(quant=quant, kv_capacity=1024, max_chunk_rows=64)
    ref = hip.HipForward(shape, w, **kw)
    want = run(ref, prompt, 24, 64)
    ref.close()

    g = hip.HipForward(shape, w, **kw)
    early_clone = g.clone()
    for l, names in evict:
        for n in names:
            assert g.evict_unit(unit(l, n))
    for l, names in evict:
        for n in names:
            assert g.unit_tier(unit(l, n)) == 2
            assert g.evict_unit(unit(l, n))  # already there: still a known unit
    evicted = {(l, n) for l, names in evict for n in names}
    resident = [(l, "mlp.up_proj") for l in range(shape.num_layers) if (l, "mlp.up_proj") not in evicted]
    for l, n in resident:
        assert g.unit_tier(unit(l, n)) == 1
    for bad in ("model.embed_tokens.weight", "model.norm.weight", f"model.layers.{shape.num_layers}.mlp.up_proj.weight",
                "model.layers.01.mlp.up_proj.weight", "model.layers.0.input_layernorm.weight", "nonsense"):
        assert not g.evict_unit(bad), bad
        assert not g.page_in_unit(bad, 0), bad
        assert g.unit_tier(bad) == 0, bad

    for model in (g, early_clone):
        got = run(model, prompt, 24, 64)
        assert np.array_equal(bits(got[0]), bits(want[0]))
        assert got[1] == want[1]
        assert np.array_equal(bits(got[2]), bits(want[2]))
    # Other chunkings and a clone made while units are evicted.
    late_clone = g.clone()
    got = run(late_clone, prompt, 8, 32)
    assert got[1] == want[1][:9]

    # Page everything back in: the same bits again, on the graph path.
    for l, names in evict:
        for n in names:
            assert g.page_in_unit(unit(l, n), 0)
            assert g.unit_tier(unit(l, n)) == 1
    g.clear_cache()
    got = run(g, prompt, 24, 64)
    assert np.array_equal(bits(got[0]), bits(want[0]))
    assert got[1] == want[1]
    assert np.array_equal(bits(got[2]), bits(want[2]))
    for m in (g, early_clone, late_clone):
        m.close()


def test_page_in_restores_the_persistent_decode(hip, monkeypatch):
    """After evict -> page-in the weights sit at new device addresses; the
    persistent kernel's layer table and the decode graphs follow them."""
    monkeypatch.delenv("CHEETAH_HIP_FUSED", raising=False)
    shape = configs.TINY_QWEN2
    w = weights(shape)
    prompt = synth.make_tokens(shape.vocab_size, 100, seed=22)
    ref = hip.HipForward(shape, w, kv_capacity=1024, max_chunk_rows=64)
    want = run(ref, prompt, 40, 64)
    ref.close()
    g = hip.HipForward(shape, w, kv_capacity=1024, max_chunk_rows=64)
    run(g, prompt, 40, 64)  # builds the table and graphs at the first addresses
    for l in range(shape.num_layers):
        for n in ALL:
            assert g.evict_unit(unit(l, n))
    for l in range(shape.num_layers):
        for n in ALL:
            assert g.page_in_unit(unit(l, n), 1)
    g.clear_cache()
    got = run(g, prompt, 40, 64)
    assert np.array_equal(bits(got[0]), bits(want[0]))
    assert got[1] == want[1]
    assert np.array_equal(bits(got[2]), bits(want[2]))
    g.close()


@pytest.mark.parametrize("quant", [None, "q8"])
def test_prepared_dir_with_ant_plan(hip, tmp_path, quant, monkeypatch):
    """A prepared directory (units manifest + safetensors shards + config.json)
    loads into the same model as the in-memory weights, and an Ant plan that
    places a layer in RAM starts it evicted with the same logits."""
    from cheetah_amd import prepared
    monkeypatch.setenv("CHEETAH_HIP_FUSED", "0")
    shape = configs.TINY_LLAMA
    w = weights(shape)
    prepared.write_prepared(str(tmp_path), w, prepared.hf_config(shape), shards=2)
    prompt = synth.make_tokens(shape.vocab_size, 90, seed=23)
    kw = dict(quant=quant, kv_capacity=512, max_chunk_rows=64)
    ref = hip.HipForward(shape, w, **kw)
    want = run(ref, prompt, 16, 64)
    ref.close()
    plan = {unit(1, n): "ram" for n in ALL}
    plan[unit(0, "mlp.up_proj")] = "vram"
    for p in (None, plan):
        g = prepared.load(str(tmp_path), plan=p, **kw)
        assert g.shape.replace(name=shape.name) == shape
        assert g.unit_tier(unit(1, "mlp.down_proj")) == (2 if p else 1)
        assert g.unit_tier(unit(0, "mlp.up_proj")) == 1
        got = run(g, prompt, 16, 64)
        assert np.array_equal(bits(got[0]), bits(want[0]))
        assert got[1] == want[1]
        assert np.array_equal(bits(got[2]), bits(want[2]))
        g.close()
