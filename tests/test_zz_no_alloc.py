"""cheetah_hip_attention_noalloc (no device allocation: split partials in a
fixed per-GPU scratch array) against cheetah_hip_attention, the entry point
it mirrors. Same kernels and split choice, so the outputs must be identical
bit for bit. Two calls in a row on the same scratch, the second smaller (a
stale larger call's partials must not leak into it), decode and a
prefill chunk, and a call too large for the scratch rejected with an error.
"""
import numpy as np
import pytest

from cheetah_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from cheetah_amd import hip as h
    h.init(0)
    return h


def _case(seed, q_heads, kv_heads, hd, ctx, rows):
    rng = np.random.default_rng(seed)
    k = synth.f32_to_bf16(rng.standard_normal((ctx, kv_heads, hd)).astype(np.float32))
    v = synth.f32_to_bf16(rng.standard_normal((ctx, kv_heads, hd)).astype(np.float32))
    q = rng.standard_normal((rows, q_heads * hd)).astype(np.float32)
    return k, v, q


@pytest.mark.parametrize("first,second", [
    # (q_heads, kv_heads, head_dim, context, rows): decode, larger then smaller
    ((32, 8, 128, 16384, 1), (32, 8, 128, 1000, 1)),
    # prefill chunks (matrix-core path with absolute splits), then decode
    ((32, 8, 128, 4608, 512), (14, 2, 64, 700, 1)),
    ((14, 2, 64, 3000, 200), (28, 4, 128, 1100, 37)),
])
def test_noalloc_matches_attention_on_two_calls(hip, first, second):
    for i, (qh, kvh, hd, ctx, rows) in enumerate((first, second)):
        k, v, q = _case(1000 * i + ctx, qh, kvh, hd, ctx, rows)
        kp, vp, table = hip.paged_kv(k, v, seed=ctx)
        ref = hip.attention(q, kp, vp, table, qh, rows, ctx - rows)
        got = hip.attention(q, kp, vp, table, qh, rows, ctx - rows, noalloc=True)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (i, qh, kvh, hd, ctx, rows)


def test_noalloc_rejects_partials_beyond_the_scratch(hip):
    # 1024 rows x 64 heads x 5 absolute splits x 130 floats = 42.6M floats
    # > the 12M-float scratch: an error sentence, no launch.
    qh, kvh, hd, ctx, rows = 64, 8, 128, 5000, 1024
    k = np.zeros((ctx, kvh, hd), np.uint16)
    q = np.zeros((rows, qh * hd), np.float32)
    kp, vp, table = hip.paged_kv(k, k, seed=1)
    with pytest.raises(hip.HipError, match="attention_noalloc needs"):
        hip.attention(q, kp, vp, table, qh, rows, ctx - rows, noalloc=True)
