"""A prepared model directory served by the HIP backend.

The native backend's load path for the qwen2 / llama families, restated:

- ``open_units``: ``MmapWeightStore::open`` (src/chat/native/store.rs:74-160).
  The units manifest ``cheetah_units.json`` lists one entry per weight tensor
  (unit_id, dtype, shape, bytes, source_file, source_offset, layer_id). Shards
  sit under ``.cheetah/weights/`` in safetensors layout: an 8-byte
  little-endian header length, the JSON header, then the payload. Unit
  offsets count from the payload start. Entries without a unit id or source
  file are skipped (store.rs:89-91). Every unit is a read-only memory map of
  its bytes, so nothing is read before the upload.
- ``resolve_shape``: ``DecoderConfig::resolve`` (src/chat/native/decoder.rs:
  255-480). ``config.json`` fields come first, then the manifest's shapes,
  then the family constants and (hidden, vocab) profiles
  (registrations/qwen2.rs:63-80, registrations/llama.rs:67-83).
- ``load``: uploads every unit into a ``HipForward``. An optional Ant plan
  (unit id -> tier name) is applied after the upload. Units planned outside
  ``vram`` are evicted to pinned host memory and streamed per layer
  (engine.rs:1210-1226 applies a plan the same way, through
  ``AntTierControl``).
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

from . import configs

UNITS_FILENAME = "cheetah_units.json"  # ant.rs:39

# Family constants (rope theta, RMS eps, tied head) and the (hidden, vocab)
# -> (q heads, kv heads, head dim) profiles used when config.json is absent.
FAMILIES = {
    "qwen2": (configs.FAMILY_QWEN2, 1_000_000.0, 1e-6, True,
              {(896, 151936): (14, 2, 64), (1536, 151936): (12, 2, 128), (3584, 152064): (28, 4, 128)}),
    "llama": (configs.FAMILY_LLAMA, 10_000.0, 1e-5, False,
              {(2048, 128256): (32, 8, 64), (3072, 128256): (24, 8, 128), (4096, 128256): (32, 8, 128),
               (4096, 32000): (32, 32, 128)}),
}

_DTYPES = {"BF16": np.uint16, "bf16": np.uint16, "F16": np.float16, "f16": np.float16, "F32": np.float32,
           "f32": np.float32}


class PreparedError(ValueError):
    pass


def read_manifest(model_dir: str) -> list:
    path = os.path.join(model_dir, UNITS_FILENAME)
    try:
        with open(path, "rb") as f:
            raw = f.read()
    except OSError as e:
        raise PreparedError(f"Failed to read {path}: {e}") from None
    try:
        units = json.loads(raw)
    except ValueError as e:
        raise PreparedError(f"Invalid Ant units manifest: {e}") from None
    if not isinstance(units, list):
        raise PreparedError("Ant units manifest must be a JSON array.")
    if not units:
        raise PreparedError("Ant units manifest is empty; run `cheetah init` first.")
    return units


def open_units(model_dir: str) -> tuple[dict, dict]:
    """unit id -> read-only array over the unit's bytes (BF16 as uint16), and
    unit id -> layer id."""
    weights_dir = os.path.join(model_dir, ".cheetah", "weights")
    shards = {}  # source_file -> (path, payload start, size)
    arrays, layers = {}, {}
    for u in read_manifest(model_dir):
        unit_id, source = u.get("unit_id") or "", u.get("source_file") or ""
        if not unit_id or not source:
            continue
        if source not in shards:
            path = os.path.join(weights_dir, source)
            try:
                size = os.path.getsize(path)
                with open(path, "rb") as f:
                    head = f.read(8)
            except OSError as e:
                raise PreparedError(f"Failed to open {path}: {e}") from None
            if len(head) < 8:
                raise PreparedError(f"Shard {path} is too small for a header.")
            start = 8 + struct.unpack("<Q", head)[0]
            if start > size:
                raise PreparedError(f"Shard {path} header exceeds the file size.")
            shards[source] = (path, start, size)
        path, start, size = shards[source]
        dtype = u.get("dtype", "f32")
        if dtype not in _DTYPES:
            raise PreparedError(f"HIP backend does not support dtype {dtype} for unit {unit_id}.")
        nbytes, offset = int(u.get("bytes", 0)), int(u.get("source_offset", 0))
        if start + offset + nbytes > size:
            raise PreparedError(f"Unit {unit_id} exceeds the bounds of shard {source}.")
        shape = tuple(int(d) for d in u.get("shape", []))
        dt = np.dtype(_DTYPES[dtype])
        if int(np.prod(shape, dtype=np.int64)) * dt.itemsize != nbytes:
            raise PreparedError(f"Unit {unit_id}: {nbytes} bytes do not match its {dtype} shape {list(shape)}.")
        arrays[unit_id] = np.memmap(path, dtype=dt, mode="r", offset=start + offset, shape=shape)
        layers[unit_id] = int(u.get("layer_id", 0))
    return arrays, layers


def resolve_shape(model_dir: str, units: dict, layers: dict, family: str | None = None) -> configs.DecoderShape:
    cfg_path = os.path.join(model_dir, "config.json")
    raw = {}
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            raw = json.load(f)
    family = family or raw.get("model_type")
    if family not in FAMILIES:
        raise PreparedError(f"HIP backend: model family {family!r} is not served (qwen2 and llama are).")
    fam, theta, eps, tied, profiles = FAMILIES[family]

    def field(name, kind):
        v = raw.get(name)
        if kind is bool:
            return v if isinstance(v, bool) else None
        if isinstance(v, bool):
            return None
        if kind is float:  # serde's as_f64 takes integers too
            return float(v) if isinstance(v, (int, float)) else None
        return v if isinstance(v, int) and v >= 0 else None  # as_u64: non-negative integers only

    embed = units.get("model.embed_tokens.weight")
    if embed is None:
        raise PreparedError("HIP backend: units manifest has no embedding tensor.")
    if embed.ndim != 2:
        raise PreparedError("HIP backend: unexpected embedding shape in the units manifest.")
    hidden = field("hidden_size", int) or embed.shape[1]
    vocab = field("vocab_size", int) or embed.shape[0]
    num_layers = field("num_hidden_layers", int) or max(max(layers.values(), default=0) + 1, 1)
    q = units.get("model.layers.0.self_attn.q_proj.weight")
    k = units.get("model.layers.0.self_attn.k_proj.weight")
    if q is None:
        raise PreparedError("HIP backend: units manifest has no model.layers.0.self_attn.q_proj.weight tensor.")
    if k is None:
        raise PreparedError("HIP backend: units manifest has no k_proj tensor.")
    gate = units.get("model.layers.0.mlp.gate_proj.weight")
    inter = field("intermediate_size", int) or (gate.shape[0] if gate is not None else 0)
    if not inter:
        raise PreparedError("HIP backend: cannot resolve the intermediate size from config.json or the units manifest.")
    use_sw = field("use_sliding_window", bool)
    sliding = (field("sliding_window", int) or 0) if (use_sw is None or use_sw) else 0
    q_heads = field("num_attention_heads", int)
    if q_heads is not None:
        head_dim = field("head_dim", int) or (profiles.get((hidden, vocab)) or (0, 0, q.shape[0] // max(q_heads, 1)))[2]
        kv_heads = field("num_key_value_heads", int)
        if kv_heads is None:
            kv_heads = k.shape[0] // head_dim if k.shape[0] % head_dim == 0 else q_heads
    elif (hidden, vocab) in profiles:
        q_heads, kv_heads, head_dim = profiles[(hidden, vocab)]
    else:
        raise PreparedError(f"HIP backend: cannot determine the attention head layout for hidden size {hidden}; "
                            "provide config.json or extend the family profiles.")
    r_eps, r_theta, r_tied = field("rms_norm_eps", float), field("rope_theta", float), field("tie_word_embeddings", bool)
    return configs.DecoderShape(
        name=os.path.basename(os.path.normpath(model_dir)), family=fam, num_layers=num_layers, hidden_size=hidden,
        q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, intermediate_size=inter, vocab_size=vocab,
        rope_theta=float(r_theta if r_theta is not None else theta), rms_eps=float(r_eps if r_eps is not None else eps),
        tie_word_embeddings=r_tied if r_tied is not None else tied,
        qkv_bias="model.layers.0.self_attn.q_proj.bias" in units, sliding_window=sliding)


def load(model_dir: str, family: str | None = None, quant=None, kv_capacity: int = 0, max_chunk_rows: int = 0,
         kv: str = "bf16", plan: dict | None = None):
    """HipForward over a prepared directory; ``plan`` maps unit ids to Ant
    tiers ("vram", "ram", "disk"); units outside "vram" start evicted."""
    from . import hip

    units, layers = open_units(model_dir)
    shape = resolve_shape(model_dir, units, layers, family)
    g = hip.HipForward(shape, units, quant=quant, kv_capacity=kv_capacity, max_chunk_rows=max_chunk_rows, kv=kv)
    for unit_id, tier in (plan or {}).items():
        if tier != "vram":
            g.evict_unit(unit_id)
    return g


def write_prepared(model_dir: str, weights: dict, config: dict | None = None, shards: int = 2,
                   layer_of=None) -> None:
    """Writes ``weights`` (unit id -> array; uint16 = BF16) as a prepared
    directory in the layout ``open_units`` reads: ``shards`` safetensors
    files under .cheetah/weights/ and the units manifest. For fixtures."""
    wdir = os.path.join(model_dir, ".cheetah", "weights")
    os.makedirs(wdir, exist_ok=True)
    names = list(weights)
    per = -(-len(names) // max(shards, 1))
    manifest = []
    kinds = {np.dtype(np.uint16): "BF16", np.dtype(np.float16): "F16", np.dtype(np.float32): "F32"}
    for s in range(0, len(names), per):
        group = names[s:s + per]
        fname = f"model-{s // per + 1:05d}-of-{-(-len(names) // per):05d}.safetensors"
        header, off = {}, 0
        for n in group:
            a = np.ascontiguousarray(weights[n])
            header[n] = {"dtype": kinds[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
            manifest.append({"unit_id": n, "name": n, "dtype": kinds[a.dtype], "shape": list(a.shape),
                             "bytes": a.nbytes, "source_file": fname, "source_offset": off, "shard": fname,
                             "layer_id": layer_of(n) if layer_of else _layer_id(n)})
            off += a.nbytes
        blob = json.dumps(header).encode()
        blob += b" " * (-len(blob) % 8)
        with open(os.path.join(wdir, fname), "wb") as f:
            f.write(struct.pack("<Q", len(blob)))
            f.write(blob)
            for n in group:
                f.write(np.ascontiguousarray(weights[n]).tobytes())
    with open(os.path.join(model_dir, UNITS_FILENAME), "w") as f:
        json.dump(manifest, f)
    if config is not None:
        with open(os.path.join(model_dir, "config.json"), "w") as f:
            json.dump(config, f)


def _layer_id(unit_id: str) -> int:
    """Decoder layer of a unit; 0 for embeddings, norms and the head (the
    manifest convention, ant.rs:620-624)."""
    parts = unit_id.split(".")
    if len(parts) > 2 and parts[0] == "model" and parts[1] == "layers" and parts[2].isdigit():
        return int(parts[2])
    return 0


def hf_config(shape: configs.DecoderShape) -> dict:
    """config.json fields of a decoder shape (the ones resolve_shape reads)."""
    return {"model_type": "qwen2" if shape.family == configs.FAMILY_QWEN2 else "llama",
            "hidden_size": shape.hidden_size, "num_hidden_layers": shape.num_layers,
            "num_attention_heads": shape.q_heads, "num_key_value_heads": shape.kv_heads, "head_dim": shape.head_dim,
            "intermediate_size": shape.intermediate_size, "vocab_size": shape.vocab_size,
            "rope_theta": shape.rope_theta, "rms_norm_eps": shape.rms_eps,
            "tie_word_embeddings": shape.tie_word_embeddings, "use_sliding_window": False, "sliding_window": 4096}
