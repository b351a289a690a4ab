"""Op-level parity of the HIP kernels against the CPU oracle, through the C-ABI.

Bars (north star): Q8/Q4 dequantized values bit-exact; GEMV / GEMM /
attention outputs within 1e-2 relative (f32 accumulation). The asserts
below are tighter where both sides accumulate in f32.
"""
import numpy as np
import pytest

from cheetah_amd import synth

pytestmark = pytest.mark.gpu

REL_BAR = 1e-2  # north-star tolerance for floating-point outputs


@pytest.fixture(scope="module")
def hip():
    from cheetah_amd import hip as h
    h.init(0)
    return h


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def random_quant(rng, fmt, rows, cols):
    """Config-3 style buffer: codes uniform over the full range, scales U[1e-3, 1e-2]."""
    scales = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)
    if fmt == "q8":
        stride = (cols + 3) // 4 * 4
        codes = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
        payload = np.zeros((rows, stride), np.uint8)
        payload[:, :cols] = codes.view(np.uint8)
    else:
        stride = ((cols + 2) // 2 + 3) // 4 * 4
        codes = rng.integers(-8, 8, (rows, cols)).astype(np.int16)
        payload = np.zeros((rows, stride), np.uint8)
        nib = (codes & 0xF).astype(np.uint8)
        payload[:, : (cols + 1) // 2] |= nib[:, 0::2]
        payload[:, : cols // 2] |= (nib[:, 1::2] << 4)
    return np.concatenate([scales.view(np.uint8), payload.reshape(-1)])


GEMV_SHAPES = [(1, 1), (3, 9), (5, 17), (64, 100), (130, 896), (259, 1000), (896, 4864), (1152, 896)]


@pytest.mark.parametrize("fmt", ["bf16", "q8", "q4"])
@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_gemv_matches_oracle(hip, oracle, fmt, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    x = rng.standard_normal(cols).astype(np.float32)
    if fmt == "bf16":
        w = synth.f32_to_bf16(rng.standard_normal((rows, cols)).astype(np.float32))
        ref = oracle.gemv(w, x)
        wd = hip.DeviceBuffer.from_array(w)
    else:
        buf = random_quant(rng, fmt, rows, cols)
        ref = oracle.gemv_quant(buf, rows, cols, x, fmt)
        wd = hip.DeviceBuffer.from_array(buf)
    got = hip.gemv(wd, fmt, rows, cols, x)
    assert rel_err(got, ref) < 1e-5 < REL_BAR


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols", [(3, 9), (4096, 4096), (4096, 14336), (14336, 4096)])
def test_config3_gemv_shapes(hip, oracle, fmt, rows, cols):
    rng = np.random.default_rng(7)
    buf = random_quant(rng, fmt, rows, cols)
    x = synth.bf16_to_f32(synth.f32_to_bf16(rng.standard_normal(cols).astype(np.float32)))
    ref = oracle.gemv_quant(buf, rows, cols, x, fmt)
    got = hip.gemv(hip.DeviceBuffer.from_array(buf), fmt, rows, cols, x)
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols", [(3, 9), (8, 64), (37, 1001), (256, 4096)])
def test_quantize_and_dequant_bit_exact(hip, oracle, fmt, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = synth.f32_to_bf16((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    w[0, :] = 0  # zero row: scale 1.0
    if rows > 2:  # exact ties: max|w| = 7 * 2^k makes w/scale hit .5 exactly
        w[1, :4] = synth.f32_to_bf16(np.array([7.0, 2.5, -2.5, 0.5], np.float32))
    values = synth.bf16_to_f32(w).reshape(rows, cols)
    ref = oracle.quantize(values, fmt)
    got = hip.quantize(w, fmt)
    assert np.array_equal(got, ref)
    deq = hip.dequant(got, fmt, rows, cols)
    assert np.array_equal(deq.view(np.uint32), oracle.dequant(ref, rows, cols, fmt).view(np.uint32))


@pytest.mark.parametrize("fmt", ["bf16", "q8", "q4"])
@pytest.mark.parametrize("n,rows,cols", [(1, 5, 9), (7, 259, 100), (64, 128, 896), (130, 300, 1000),
                                         (128, 1152, 896)])
def test_gemm_matches_oracle(hip, oracle, fmt, n, rows, cols):
    rng = np.random.default_rng(n * 7 + rows)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    if fmt == "bf16":
        w = synth.f32_to_bf16(rng.standard_normal((rows, cols)).astype(np.float32))
        ref = oracle.gemm_bf16(w, x)
        wd = hip.DeviceBuffer.from_array(w)
    else:
        buf = random_quant(rng, fmt, rows, cols)
        ref = np.stack([oracle.gemv_quant(buf, rows, cols, x[t], fmt) for t in range(n)])
        wd = hip.DeviceBuffer.from_array(buf)
    got = hip.gemm(wd, fmt, rows, cols, x)
    assert rel_err(got, ref) < 1e-4 < REL_BAR


@pytest.mark.parametrize("fmt", ["bf16", "q4"])
def test_config3_gemm_prefill_chunk(hip, oracle, fmt):
    # N = 512 against 4096 x 4096 (the prefill-chunk case of the GEMV/GEMM op).
    rng = np.random.default_rng(11)
    rows = cols = 4096
    n = 512
    x = synth.bf16_to_f32(synth.f32_to_bf16(rng.standard_normal((n, cols)).astype(np.float32))).reshape(n, cols)
    if fmt == "bf16":
        w = synth.f32_to_bf16(rng.standard_normal((rows, cols)).astype(np.float32))
        ref = oracle.gemm_bf16(w, x)
        wd = hip.DeviceBuffer.from_array(w)
    else:
        buf = random_quant(rng, fmt, rows, cols)
        sel = np.arange(0, n, 37)
        ref = np.stack([oracle.gemv_quant(buf, rows, cols, x[t], fmt) for t in sel])
        wd = hip.DeviceBuffer.from_array(buf)
    got = hip.gemm(wd, fmt, rows, cols, x)
    if fmt != "bf16":
        got = got[sel]
    assert rel_err(got, ref) < 1e-4


@pytest.mark.parametrize("fmt", ["bf16", "q8", "q4"])
def test_gemm_bits_independent_of_token_count(hip, fmt):
    """4096 x 4096 weights (16 accumulation chunks of 256) on 256 CUs: 1,024
    tokens fold K in registers on 8-wave blocks, 512 tokens run the two chunk
    halves as separate 8-wave blocks (half sums folded by the reduce), 128
    tokens one block per chunk (all 16 sums folded by the reduce). Each path
    folds the chunks as two halves, so a token's outputs are the same bits in
    all three (a prompt's results do not depend on how it is chunked)."""
    rng = np.random.default_rng(5)
    rows = cols = 4096
    x = rng.standard_normal((1024, cols)).astype(np.float32)
    if fmt == "bf16":
        wd = hip.DeviceBuffer.from_array(synth.f32_to_bf16(rng.standard_normal((rows, cols)).astype(np.float32)))
    else:
        wd = hip.DeviceBuffer.from_array(random_quant(rng, fmt, rows, cols))

    def bits(a):
        return np.ascontiguousarray(a, np.float32).view(np.uint32)

    y1024 = hip.gemm(wd, fmt, rows, cols, x)
    y512 = hip.gemm(wd, fmt, rows, cols, x[:512])
    y128 = hip.gemm(wd, fmt, rows, cols, x[:128])
    assert np.array_equal(bits(y1024[:512]), bits(y512))
    assert np.array_equal(bits(y512[:128]), bits(y128))
    assert np.isfinite(y1024).all() and np.abs(y1024).max() > 0


def _attn_case(rng, q_heads, kv_heads, hd, ctx, rows):
    k = synth.f32_to_bf16(rng.standard_normal((ctx, kv_heads, hd)).astype(np.float32))
    v = synth.f32_to_bf16(rng.standard_normal((ctx, kv_heads, hd)).astype(np.float32))
    q = rng.standard_normal((rows, q_heads * hd)).astype(np.float32)
    return k, v, q


@pytest.mark.parametrize("q_heads,kv_heads,hd", [(14, 2, 64), (32, 8, 128), (28, 4, 128), (4, 4, 64), (8, 1, 64)])
@pytest.mark.parametrize("ctx", [1, 63, 64, 65, 1000, 4096])
def test_attention_decode_matches_oracle(hip, oracle, q_heads, kv_heads, hd, ctx):
    rng = np.random.default_rng(ctx + q_heads)
    k, v, q = _attn_case(rng, q_heads, kv_heads, hd, ctx, 1)
    kp, vp, table = hip.paged_kv(k, v, seed=ctx)
    got = hip.attention(q, kp, vp, table, q_heads, 1, ctx - 1)[0]
    ref = oracle.attention(synth.bf16_to_f32(k), synth.bf16_to_f32(v), q[0], q_heads, kv_heads, hd, ctx - 1)
    assert np.max(np.abs(got - ref)) < 1e-4


@pytest.mark.parametrize("q_heads,kv_heads,hd,offset,rows", [(14, 2, 64, 0, 37), (32, 8, 128, 100, 70),
                                                            (28, 4, 128, 4000, 9)])
def test_attention_prefill_rows_match_oracle(hip, oracle, q_heads, kv_heads, hd, offset, rows):
    rng = np.random.default_rng(offset + rows)
    ctx = offset + rows
    k, v, q = _attn_case(rng, q_heads, kv_heads, hd, ctx, rows)
    kp, vp, table = hip.paged_kv(k, v, seed=rows)
    got = hip.attention(q, kp, vp, table, q_heads, rows, offset)
    kf, vf = synth.bf16_to_f32(k), synth.bf16_to_f32(v)
    for i in range(rows):
        pos = offset + i
        ref = oracle.attention(kf[: pos + 1], vf[: pos + 1], q[i], q_heads, kv_heads, hd, pos)
        assert np.max(np.abs(got[i] - ref)) < 1e-4, i


def test_attention_two_token_gqa_kat(hip):
    # native.rs:2017-2033 closed form, through the paged kernel (hd padded to
    # 64 with zeros; zero dims change neither scores nor outputs... except the
    # 1/sqrt(head_dim) scale, so the expected weights use hd = 64).
    hd = 64
    k = np.zeros((2, 1, hd), np.float32)
    v = np.zeros((2, 1, hd), np.float32)
    k[0, 0, 0] = 1.0
    k[1, 0, 1] = 1.0
    v[0, 0, :2] = [2.0, 3.0]
    v[1, 0, :2] = [5.0, 7.0]
    q = np.zeros((1, 2 * hd), np.float32)
    q[0, 0] = 1.0
    q[0, hd + 1] = 1.0
    kp, vp, table = hip.paged_kv(synth.f32_to_bf16(k), synth.f32_to_bf16(v))
    out = hip.attention(q, kp, vp, table, 2, 1, 1)[0]
    w = 1.0 / (1.0 + np.exp(-1.0 / np.sqrt(hd)))
    exp0 = [2 * w + 5 * (1 - w), 3 * w + 7 * (1 - w)]
    exp1 = [2 * (1 - w) + 5 * w, 3 * (1 - w) + 7 * w]
    assert np.allclose(out[:2], exp0, atol=1e-5) and np.allclose(out[hd:hd + 2], exp1, atol=1e-5)
