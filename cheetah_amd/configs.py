"""Decoder shapes served by the HIP backend.

The fields mirror ``DecoderConfig`` (src/chat/native/decoder.rs:29-85) as
resolved for the two families on the hot path: qwen2
(src/chat/registrations/qwen2.rs:67-85: theta 1e6, eps 1e-6, tied head,
q/k/v biases) and llama (src/chat/registrations/llama.rs:64-82: eps 1e-5,
untied head, no biases).
"""
from __future__ import annotations

import dataclasses

FAMILY_QWEN2 = 0
FAMILY_LLAMA = 1


@dataclasses.dataclass(frozen=True)
class DecoderShape:
    name: str
    family: int
    num_layers: int
    hidden_size: int
    q_heads: int
    kv_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    rope_theta: float
    rms_eps: float
    tie_word_embeddings: bool
    qkv_bias: bool
    sliding_window: int = 0

    @property
    def q_dim(self) -> int:
        return self.q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def rotary_dim(self) -> int:
        return self.head_dim

    def linear_units(self, layer: int):
        """(unit id, rows, cols) of every linear projection of one layer."""
        p = f"model.layers.{layer}."
        h, i = self.hidden_size, self.intermediate_size
        return [
            (p + "self_attn.q_proj.weight", self.q_dim, h),
            (p + "self_attn.k_proj.weight", self.kv_dim, h),
            (p + "self_attn.v_proj.weight", self.kv_dim, h),
            (p + "self_attn.o_proj.weight", h, self.q_dim),
            (p + "mlp.gate_proj.weight", i, h),
            (p + "mlp.up_proj.weight", i, h),
            (p + "mlp.down_proj.weight", h, i),
        ]

    def linear_params(self) -> int:
        return sum(r * c for layer in range(self.num_layers) for _, r, c in self.linear_units(layer))

    def head_params(self) -> int:
        return self.vocab_size * self.hidden_size

    def replace(self, **kw) -> "DecoderShape":
        return dataclasses.replace(self, **kw)


# Qwen2-0.5B architecture (qwen2.rs:74 profile (896, 151936, 14, 2, 64)).
QWEN2_0_5B = DecoderShape(
    name="qwen2-0.5b", family=FAMILY_QWEN2, num_layers=24, hidden_size=896, q_heads=14, kv_heads=2,
    head_dim=64, intermediate_size=4864, vocab_size=151936, rope_theta=1e6, rms_eps=1e-6,
    tie_word_embeddings=True, qkv_bias=True)

# Llama-3-8B architecture (llama.rs:75 profile (4096, 128256, 32, 8, 128)), theta 5e5.
LLAMA3_8B = DecoderShape(
    name="llama3-8b", family=FAMILY_LLAMA, num_layers=32, hidden_size=4096, q_heads=32, kv_heads=8,
    head_dim=128, intermediate_size=14336, vocab_size=128256, rope_theta=5e5, rms_eps=1e-5,
    tie_word_embeddings=False, qkv_bias=False)

# Qwen2-7B architecture (qwen2.rs:76 profile (3584, 152064, 28, 4, 128)), untied.
QWEN2_7B = DecoderShape(
    name="qwen2-7b", family=FAMILY_QWEN2, num_layers=28, hidden_size=3584, q_heads=28, kv_heads=4,
    head_dim=128, intermediate_size=18944, vocab_size=152064, rope_theta=1e6, rms_eps=1e-6,
    tie_word_embeddings=False, qkv_bias=True)

# Small shapes for tests that must finish in seconds on the CPU oracle.
TINY_QWEN2 = DecoderShape(
    name="tiny-qwen2", family=FAMILY_QWEN2, num_layers=2, hidden_size=128, q_heads=4, kv_heads=2,
    head_dim=64, intermediate_size=352, vocab_size=1000, rope_theta=1e6, rms_eps=1e-6,
    tie_word_embeddings=True, qkv_bias=True)

TINY_LLAMA = DecoderShape(
    name="tiny-llama", family=FAMILY_LLAMA, num_layers=2, hidden_size=256, q_heads=8, kv_heads=2,
    head_dim=128, intermediate_size=704, vocab_size=1203, rope_theta=5e5, rms_eps=1e-5,
    tie_word_embeddings=False, qkv_bias=False)

SHAPES = {s.name: s for s in (QWEN2_0_5B, LLAMA3_8B, QWEN2_7B, TINY_QWEN2, TINY_LLAMA)}
