"""Prepared-directory loading on the CPU: the units manifest and safetensors
shards (MmapWeightStore::open, src/chat/native/store.rs:74-160) and the
config resolution order config.json -> manifest shapes -> family constants
(DecoderConfig::resolve, src/chat/native/decoder.rs:255-480)."""
import json
import os

import numpy as np
import pytest

from cheetah_amd import configs, prepared, synth


@pytest.fixture(scope="module")
def tiny_weights():
    return {s.name: synth.make_weights(s) for s in (configs.TINY_QWEN2, configs.TINY_LLAMA)}


@pytest.mark.parametrize("shape", [configs.TINY_QWEN2, configs.TINY_LLAMA], ids=lambda s: s.name)
def test_units_round_trip_and_full_config(tmp_path, tiny_weights, shape):
    w = tiny_weights[shape.name]
    prepared.write_prepared(str(tmp_path), w, prepared.hf_config(shape), shards=3)
    assert len(os.listdir(tmp_path / ".cheetah" / "weights")) == 3
    units, layers = prepared.open_units(str(tmp_path))
    assert set(units) == set(w)
    for name, arr in w.items():
        assert units[name].dtype == np.uint16 and np.array_equal(units[name], arr), name
    assert layers["model.layers.1.mlp.up_proj.weight"] == 1
    assert layers["model.embed_tokens.weight"] == 0 and layers["model.norm.weight"] == 0
    got = prepared.resolve_shape(str(tmp_path), units, layers)
    assert got.replace(name=shape.name) == shape


def test_partial_config_falls_back_to_manifest_and_family(tmp_path, tiny_weights):
    shape = configs.TINY_QWEN2
    prepared.write_prepared(str(tmp_path), tiny_weights[shape.name], {"model_type": "qwen2",
                                                                     "num_attention_heads": shape.q_heads})
    units, layers = prepared.open_units(str(tmp_path))
    got = prepared.resolve_shape(str(tmp_path), units, layers)
    # hidden/vocab from the embedding, layers from the highest layer id,
    # head_dim = q rows / heads, kv heads = k rows / head_dim, intermediate
    # from gate rows; theta, eps and the tied head from the qwen2 constants.
    assert (got.hidden_size, got.vocab_size, got.num_layers) == (128, 1000, 2)
    assert (got.q_heads, got.kv_heads, got.head_dim, got.intermediate_size) == (4, 2, 64, 352)
    assert (got.rope_theta, got.rms_eps, got.tie_word_embeddings, got.qkv_bias) == (1e6, 1e-6, True, True)


def test_family_profile_without_config():
    # Shapes only (zero-stride views): (hidden, vocab) = (4096, 128256)
    # selects the Llama-3-8B profile, 32 q / 8 kv heads of 128.
    def fake(*shape):
        return np.lib.stride_tricks.as_strided(np.zeros(1, np.uint16), shape=shape, strides=(0,) * len(shape))
    units = {"model.embed_tokens.weight": fake(128256, 4096),
             "model.layers.0.self_attn.q_proj.weight": fake(4096, 4096),
             "model.layers.0.self_attn.k_proj.weight": fake(1024, 4096),
             "model.layers.0.mlp.gate_proj.weight": fake(14336, 4096)}
    got = prepared.resolve_shape("/nonexistent-dir", units, {"model.layers.31.mlp.up_proj.weight": 31}, "llama")
    assert (got.q_heads, got.kv_heads, got.head_dim, got.num_layers, got.intermediate_size) == (32, 8, 128, 32, 14336)
    assert (got.rope_theta, got.rms_eps, got.tie_word_embeddings) == (10000.0, 1e-5, False)
    units["model.embed_tokens.weight"] = fake(1000, 4096)
    with pytest.raises(prepared.PreparedError, match="cannot determine the attention head layout"):
        prepared.resolve_shape("/nonexistent-dir", units, {}, "llama")


def test_sliding_window_resolution(tmp_path, tiny_weights):
    shape = configs.TINY_QWEN2
    cfg = prepared.hf_config(shape)
    prepared.write_prepared(str(tmp_path), tiny_weights[shape.name], dict(cfg, use_sliding_window=True))
    units, layers = prepared.open_units(str(tmp_path))
    assert prepared.resolve_shape(str(tmp_path), units, layers).sliding_window == 4096
    with open(tmp_path / "config.json", "w") as f:
        json.dump(dict(cfg, use_sliding_window=False), f)
    assert prepared.resolve_shape(str(tmp_path), units, layers).sliding_window == 0


def _manifest(tmp_path):
    with open(tmp_path / "cheetah_units.json") as f:
        return json.load(f)


def _rewrite(tmp_path, m):
    with open(tmp_path / "cheetah_units.json", "w") as f:
        json.dump(m, f)


def test_manifest_errors(tmp_path, tiny_weights):
    shape = configs.TINY_QWEN2
    prepared.write_prepared(str(tmp_path), tiny_weights[shape.name], prepared.hf_config(shape), shards=1)
    m = _manifest(tmp_path)
    # Entries without a unit id or a source file are skipped.
    _rewrite(tmp_path, m + [{"unit_id": "", "source_file": "x"}, {"unit_id": "orphan", "source_file": ""}])
    units, _ = prepared.open_units(str(tmp_path))
    assert "orphan" not in units and len(units) == len(m)
    bad = [dict(m[0], bytes=m[0]["bytes"] * 10**6)] + m[1:]
    _rewrite(tmp_path, bad)
    with pytest.raises(prepared.PreparedError, match="exceeds the bounds of shard"):
        prepared.open_units(str(tmp_path))
    _rewrite(tmp_path, [dict(m[0], dtype="I8")] + m[1:])
    with pytest.raises(prepared.PreparedError, match="does not support dtype I8"):
        prepared.open_units(str(tmp_path))
    _rewrite(tmp_path, [dict(m[0], shape=[3, 3])] + m[1:])
    with pytest.raises(prepared.PreparedError, match="do not match"):
        prepared.open_units(str(tmp_path))
    _rewrite(tmp_path, [])
    with pytest.raises(prepared.PreparedError, match="empty"):
        prepared.open_units(str(tmp_path))
    _rewrite(tmp_path, m)
    shard = tmp_path / ".cheetah" / "weights" / m[0]["source_file"]
    shard.write_bytes(b"\x01\x02")
    with pytest.raises(prepared.PreparedError, match="too small for a header"):
        prepared.open_units(str(tmp_path))
    shard.write_bytes((1 << 40).to_bytes(8, "little"))
    with pytest.raises(prepared.PreparedError, match="header exceeds the file size"):
        prepared.open_units(str(tmp_path))
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"model_type": "gemma"}, f)
    with pytest.raises(prepared.PreparedError, match="not served"):
        prepared.resolve_shape(str(tmp_path), {}, {})
