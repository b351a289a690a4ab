"""ctypes binding of the CPU oracle (libcheetah_ref_cpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's CPU-baseline leg, always as the checker or the timed CPU
baseline, never as the product path. The library restates the arithmetic of
the reference's native CPU backend (src/chat/native/ops.rs,
src/chat/precision/{q8,q4}.rs, src/chat/registrations/{qwen2,llama}.rs).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcheetah_ref_cpu.so")

_F32P = ctypes.POINTER(ctypes.c_float)
_U8P = ctypes.POINTER(ctypes.c_uint8)
_U16P = ctypes.POINTER(ctypes.c_uint16)
_U32P = ctypes.POINTER(ctypes.c_uint32)
_U64P = ctypes.POINTER(ctypes.c_uint64)
_SZ = ctypes.c_size_t


class RefConfig(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_uint32),
        ("hidden_size", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("rotary_dim", ctypes.c_uint32),
        ("intermediate_size", ctypes.c_uint32),
        ("vocab_size", ctypes.c_uint32),
        ("tie_word_embeddings", ctypes.c_uint32),
        ("sliding_window", ctypes.c_uint32),
        ("rope_theta", ctypes.c_float),
        ("rms_eps", ctypes.c_float),
    ]


def build(force: bool = True) -> None:
    args = ["make", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(force=False)
        L = ctypes.CDLL(LIB_PATH)
        L.ref_gemv.argtypes = [ctypes.c_void_p, ctypes.c_int, _SZ, _SZ, _F32P, _F32P]
        L.ref_gemm_bf16.argtypes = [_U16P, _SZ, _SZ, _F32P, _SZ, _F32P]
        L.ref_gemv_q8.argtypes = [_U8P, _SZ, _SZ, _F32P, _F32P]
        L.ref_gemv_q4.argtypes = [_U8P, _SZ, _SZ, _F32P, _F32P]
        L.ref_q8_buffer_bytes.argtypes = [_SZ, _SZ]
        L.ref_q8_buffer_bytes.restype = _SZ
        L.ref_q4_buffer_bytes.argtypes = [_SZ, _SZ]
        L.ref_q4_buffer_bytes.restype = _SZ
        L.ref_q4_row_stride.argtypes = [_SZ]
        L.ref_q4_row_stride.restype = _SZ
        L.ref_quantize_q8.argtypes = [_F32P, _SZ, _SZ, _U8P, _SZ]
        L.ref_quantize_q4.argtypes = [_F32P, _SZ, _SZ, _U8P, _SZ]
        L.ref_q8_dequant_value.argtypes = [_U8P, _SZ, _SZ, _SZ, _SZ]
        L.ref_q8_dequant_value.restype = ctypes.c_float
        L.ref_q4_dequant_value.argtypes = [_U8P, _SZ, _SZ, _SZ, _SZ]
        L.ref_q4_dequant_value.restype = ctypes.c_float
        L.ref_rmsnorm.argtypes = [_F32P, _SZ, _U16P, ctypes.c_float]
        L.ref_rope_in_place.argtypes = [_F32P, _SZ, _SZ, _SZ, ctypes.c_float]
        L.ref_rope_heads.argtypes = [_F32P, _SZ, _SZ, _SZ, _SZ, ctypes.c_float]
        L.ref_silu_multiply.argtypes = [_F32P, _F32P, _SZ]
        L.ref_round_bf16.argtypes = [_F32P, _F32P, _SZ]
        L.ref_softmax.argtypes = [_F32P, _SZ]
        L.ref_attention.argtypes = [_F32P, _F32P, _SZ, _F32P, _F32P, _SZ, _SZ, _SZ, _SZ, _SZ]
        L.ref_attention_rows.argtypes = [_F32P, _F32P, _SZ, _SZ, _F32P, _F32P, _SZ, _SZ, _SZ, _SZ]
        L.ref_gemm_quant.argtypes = [_U8P, ctypes.c_uint32, _SZ, _SZ, _F32P, _SZ, _F32P]
        L.ref_set_threads.argtypes = [ctypes.c_int]
        L.ref_get_threads.restype = ctypes.c_int
        L.ref_model_create.argtypes = [ctypes.POINTER(RefConfig), ctypes.c_uint32, ctypes.c_int]
        L.ref_model_create.restype = ctypes.c_void_p
        L.ref_model_set_unit.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, _SZ, ctypes.c_int,
                                         _U64P, _SZ]
        L.ref_model_forward.argtypes = [ctypes.c_void_p, _U32P, _SZ, _SZ, _SZ, _F32P]
        L.ref_model_clear_cache.argtypes = [ctypes.c_void_p]
        L.ref_model_clone.argtypes = [ctypes.c_void_p]
        L.ref_model_clone.restype = ctypes.c_void_p
        L.ref_model_kv_len.argtypes = [ctypes.c_void_p]
        L.ref_model_kv_len.restype = _SZ
        L.ref_model_kv_snapshot.argtypes = [ctypes.c_void_p]
        L.ref_model_kv_snapshot.restype = ctypes.c_void_p
        L.ref_model_restore_kv_prefix.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _SZ]
        L.ref_snapshot_positions.argtypes = [ctypes.c_void_p]
        L.ref_snapshot_positions.restype = _SZ
        L.ref_snapshot_free.argtypes = [ctypes.c_void_p]
        L.ref_model_free.argtypes = [ctypes.c_void_p]
        L.ref_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().ref_set_threads(n)


def get_threads() -> int:
    return lib().ref_get_threads()


def gemv(weight: np.ndarray, x, dtype: str = "bf16") -> np.ndarray:
    """y = W x; weight is uint16 BF16 bits or float32, shape [rows, cols]."""
    rows, cols = weight.shape
    x = _f32(x)
    y = np.empty(rows, np.float32)
    w = np.ascontiguousarray(weight)
    lib().ref_gemv(w.ctypes.data, 1 if dtype == "bf16" else 0, rows, cols, _p(x, _F32P), _p(y, _F32P))
    return y


def gemm_bf16(weight: np.ndarray, x) -> np.ndarray:
    rows, cols = weight.shape
    x = _f32(x).reshape(-1, cols)
    n = x.shape[0]
    y = np.empty((n, rows), np.float32)
    w = np.ascontiguousarray(weight, dtype=np.uint16)
    lib().ref_gemm_bf16(_p(w, _U16P), rows, cols, _p(x, _F32P), n, _p(y, _F32P))
    return y


def q8_buffer_bytes(rows: int, cols: int) -> int:
    return lib().ref_q8_buffer_bytes(rows, cols)


def q4_buffer_bytes(rows: int, cols: int) -> int:
    return lib().ref_q4_buffer_bytes(rows, cols)


def q4_row_stride(cols: int) -> int:
    return lib().ref_q4_row_stride(cols)


def quantize(values: np.ndarray, fmt: str) -> np.ndarray:
    values = _f32(values)
    rows, cols = values.shape
    size = q8_buffer_bytes(rows, cols) if fmt == "q8" else q4_buffer_bytes(rows, cols)
    out = np.zeros(size, np.uint8)
    fn = lib().ref_quantize_q8 if fmt == "q8" else lib().ref_quantize_q4
    rc = fn(_p(values, _F32P), rows, cols, _p(out, _U8P), size)
    if rc != 0:
        raise ValueError(lib().ref_last_error().decode())
    return out


def gemv_quant(buffer: np.ndarray, rows: int, cols: int, x, fmt: str) -> np.ndarray:
    x = _f32(x)
    y = np.empty(rows, np.float32)
    buf = np.ascontiguousarray(buffer, dtype=np.uint8)
    fn = lib().ref_gemv_q8 if fmt == "q8" else lib().ref_gemv_q4
    fn(_p(buf, _U8P), rows, cols, _p(x, _F32P), _p(y, _F32P))
    return y


def gemm_quant(buffer: np.ndarray, rows: int, cols: int, x, fmt: str) -> np.ndarray:
    """n tokens at once (x [n, cols] -> y [n, rows]); bit-identical to per-token gemv_quant."""
    x = _f32(x).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    buf = np.ascontiguousarray(buffer, dtype=np.uint8)
    lib().ref_gemm_quant(_p(buf, _U8P), 4 if fmt == "q8" else 5, rows, cols, _p(x, _F32P), x.shape[0],
                         _p(y, _F32P))
    return y


def dequant(buffer: np.ndarray, rows: int, cols: int, fmt: str) -> np.ndarray:
    """Every dequantized value scale * code (Q8Matrix/Q4Matrix::dequant_value)."""
    buf = np.ascontiguousarray(buffer, dtype=np.uint8)
    scales = buf[: rows * 4].view(np.float32)
    if fmt == "q8":
        stride = (cols + 3) // 4 * 4
        payload = buf[rows * 4:].reshape(rows, stride)[:, :cols].view(np.int8).astype(np.float32)
    else:
        stride = q4_row_stride(cols)
        payload_bytes = buf[rows * 4:].reshape(rows, stride)
        cidx = np.arange(cols)
        b = payload_bytes[:, cidx // 2]
        nib = np.where(cidx % 2 == 0, b & 0x0F, b >> 4).astype(np.int16)
        payload = np.where(nib >= 8, nib - 16, nib).astype(np.float32)
    return np.ascontiguousarray(scales[:, None] * payload, dtype=np.float32)


def rmsnorm(x, weight_bf16: np.ndarray, eps: float) -> np.ndarray:
    x = _f32(x).copy()
    w = np.ascontiguousarray(weight_bf16, dtype=np.uint16)
    lib().ref_rmsnorm(_p(x, _F32P), x.size, _p(w, _U16P), eps)
    return x


def rope_heads(values, heads: int, head_dim: int, rotary_dim: int, position: int, theta: float) -> np.ndarray:
    v = _f32(values).copy()
    lib().ref_rope_heads(_p(v, _F32P), heads, head_dim, rotary_dim, position, theta)
    return v


def round_bf16(values) -> np.ndarray:
    """The BF16-KV mode's rounding of a K/V element (nearest, ties to even),
    widened back to f32."""
    x = _f32(values).reshape(-1)
    out = np.empty_like(x)
    lib().ref_round_bf16(_p(x, _F32P), _p(out, _F32P), x.size)
    return out.reshape(np.shape(values))


def silu_multiply(gate, up) -> np.ndarray:
    g = _f32(gate).copy()
    u = _f32(up)
    lib().ref_silu_multiply(_p(g, _F32P), _p(u, _F32P), g.size)
    return g


def softmax(scores) -> np.ndarray:
    s = _f32(scores).copy()
    lib().ref_softmax(_p(s, _F32P), s.size)
    return s


def attention(keys, values, q, q_heads: int, kv_heads: int, head_dim: int, position: int,
              sliding_window: int = 0) -> np.ndarray:
    """keys/values: f32 [cache_len, kv_heads, head_dim]; q: [q_heads*head_dim]."""
    k = _f32(keys)
    v = _f32(values)
    qq = _f32(q)
    cache_len = k.size // (kv_heads * head_dim)
    out = np.zeros(q_heads * head_dim, np.float32)
    lib().ref_attention(_p(k, _F32P), _p(v, _F32P), cache_len, _p(qq, _F32P), _p(out, _F32P), q_heads, kv_heads,
                        head_dim, position, sliding_window)
    return out


def attention_rows(keys, values, q, q_heads: int, kv_heads: int, head_dim: int, offset: int,
                   sliding_window: int = 0) -> np.ndarray:
    """One chunk: keys/values f32 [offset + rows, kv_heads, head_dim], q [rows, q_heads*head_dim]; row r
    attends over the first offset + r + 1 positions."""
    k = _f32(keys)
    v = _f32(values)
    qq = _f32(q).reshape(-1, q_heads * head_dim)
    rows = qq.shape[0]
    if k.size != (offset + rows) * kv_heads * head_dim:
        raise ValueError("cache does not hold offset + rows positions")
    out = np.zeros_like(qq)
    lib().ref_attention_rows(_p(k, _F32P), _p(v, _F32P), offset, rows, _p(qq, _F32P), _p(out, _F32P), q_heads,
                             kv_heads, head_dim, sliding_window)
    return out


QUANT_CODES = {None: 0, "bf16": 0, "q8": 4, "q4": 5}


class RefModel:
    """The reference forward (qwen2.rs / llama.rs) over borrowed BF16 units."""

    def __init__(self, shape, weights: dict, quant=None, kv_bf16: bool = False, _handle=None):
        self.shape = shape
        # The library borrows the bytes (like the reference's mmap store), so
        # the contiguous arrays it was given must outlive it.
        self._weights = {name: np.ascontiguousarray(arr) for name, arr in weights.items()}
        L = lib()
        if _handle is not None:
            self._h = _handle
            return
        cfg = RefConfig(shape.num_layers, shape.hidden_size, shape.q_heads, shape.kv_heads, shape.head_dim,
                        shape.rotary_dim, shape.intermediate_size, shape.vocab_size,
                        int(shape.tie_word_embeddings), shape.sliding_window, shape.rope_theta, shape.rms_eps)
        self._h = L.ref_model_create(ctypes.byref(cfg), QUANT_CODES[quant], int(kv_bf16))
        if not self._h:
            raise ValueError(L.ref_last_error().decode())
        for name, arr in self._weights.items():
            dims = (ctypes.c_uint64 * arr.ndim)(*arr.shape)
            dtype = 1 if arr.dtype == np.uint16 else 0
            rc = L.ref_model_set_unit(self._h, name.encode(), arr.ctypes.data, arr.nbytes, dtype, dims, arr.ndim)
            if rc != 0:
                raise ValueError(L.ref_last_error().decode())

    def forward(self, tokens, offset: int, chunk_rows: int = 256) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.shape.vocab_size, np.float32)
        rc = lib().ref_model_forward(self._h, _p(toks, _U32P), toks.size, offset, chunk_rows, _p(logits, _F32P))
        if rc != 0:
            raise ValueError(lib().ref_last_error().decode())
        return logits

    def clear_cache(self) -> None:
        lib().ref_model_clear_cache(self._h)

    def clone(self) -> "RefModel":
        return RefModel(self.shape, self._weights, _handle=lib().ref_model_clone(self._h))

    def kv_len(self) -> int:
        return lib().ref_model_kv_len(self._h)

    def kv_snapshot(self):
        return RefSnapshot(lib().ref_model_kv_snapshot(self._h))

    def restore_kv_prefix(self, snapshot, positions: int) -> bool:
        return bool(lib().ref_model_restore_kv_prefix(self._h, snapshot._h, positions))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.ref_model_free(h)
            self._h = None


class RefSnapshot:
    def __init__(self, handle):
        self._h = handle

    @property
    def positions(self) -> int:
        return lib().ref_snapshot_positions(self._h)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ref_snapshot_free(self._h)
            self._h = None
