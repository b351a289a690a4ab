"""ctypes binding of libcheetah_hip.so (include/cheetah_hip.h).

This plays the role the reference's Rust FFI wrappers play for the Vulkan
C-ABI (src/native.rs:927-1937): it declares the entry points, keeps a
process-wide lock, validates lengths on the host and turns a -1 status into
an exception carrying the library's sentence (check_native_result,
native.rs:1860-1870). There is no fallback: if the library is missing or the
device is not a gfx950, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcheetah_hip.so")

FMT_BF16, FMT_Q8, FMT_Q4 = 1, 4, 5
QUANT = {None: 0, "bf16": 0, "q8": FMT_Q8, "q4": FMT_Q4}
KV_FORMATS = {"bf16": 0, "f32": 1}

_c = ctypes
_SZ = _c.c_size_t
_VP = _c.c_void_p
_U32P = _c.POINTER(_c.c_uint32)
_F32P = _c.POINTER(_c.c_float)


class HipError(RuntimeError):
    pass


class Config(_c.Structure):
    _fields_ = [(n, _c.c_uint32) for n in (
        "family", "num_layers", "hidden_size", "q_heads", "kv_heads", "head_dim", "rotary_dim",
        "intermediate_size", "vocab_size", "tie_word_embeddings", "sliding_window")] + [
        ("rope_theta", _c.c_float), ("rms_eps", _c.c_float)]


class KvView(_c.Structure):
    _fields_ = [("k_pages", _VP), ("v_pages", _VP), ("page_table", _VP), ("page_size", _c.c_uint32),
                ("kv_heads", _c.c_uint32), ("head_dim", _c.c_uint32)]


# name -> (restype, argtypes): every symbol include/cheetah_hip.h declares.
SIGNATURES = {
    "cheetah_hip_init": (_c.c_int, [_c.c_int]),
    "cheetah_hip_shutdown": (None, []),
    "cheetah_hip_device_name": (_c.c_char_p, []),
    "cheetah_hip_last_error": (_c.c_char_p, []),
    "cheetah_hip_alloc": (_VP, [_SZ]),
    "cheetah_hip_free": (_c.c_int, [_VP]),
    "cheetah_hip_upload": (_c.c_int, [_VP, _VP, _SZ]),
    "cheetah_hip_download": (_c.c_int, [_VP, _VP, _SZ]),
    "cheetah_hip_copy": (_c.c_int, [_VP, _VP, _SZ]),
    "cheetah_hip_synchronize": (_c.c_int, []),
    "cheetah_hip_gemv_bf16": (_c.c_int, [_VP, _SZ, _SZ, _VP, _VP]),
    "cheetah_hip_gemv_q8": (_c.c_int, [_VP, _SZ, _SZ, _VP, _VP]),
    "cheetah_hip_gemv_q4": (_c.c_int, [_VP, _SZ, _SZ, _VP, _VP]),
    "cheetah_hip_gemm_bf16": (_c.c_int, [_VP, _SZ, _SZ, _VP, _SZ, _VP]),
    "cheetah_hip_gemm_q8": (_c.c_int, [_VP, _SZ, _SZ, _VP, _SZ, _VP]),
    "cheetah_hip_gemm_q4": (_c.c_int, [_VP, _SZ, _SZ, _VP, _SZ, _VP]),
    "cheetah_hip_q8_buffer_bytes": (_SZ, [_SZ, _SZ]),
    "cheetah_hip_q4_buffer_bytes": (_SZ, [_SZ, _SZ]),
    "cheetah_hip_quantize_q8": (_c.c_int, [_VP, _SZ, _SZ, _VP, _SZ]),
    "cheetah_hip_quantize_q4": (_c.c_int, [_VP, _SZ, _SZ, _VP, _SZ]),
    "cheetah_hip_dequant_q8": (_c.c_int, [_VP, _SZ, _SZ, _VP]),
    "cheetah_hip_dequant_q4": (_c.c_int, [_VP, _SZ, _SZ, _VP]),
    "cheetah_hip_attention": (_c.c_int, [_VP, _c.POINTER(KvView), _c.c_uint32, _SZ, _SZ, _VP]),
    "cheetah_hip_attention_noalloc": (_c.c_int, [_VP, _c.POINTER(KvView), _c.c_uint32, _SZ, _SZ, _VP]),
    "cheetah_hip_model_create": (_VP, [_c.POINTER(Config), _c.c_uint32, _c.c_uint32, _SZ, _SZ]),
    "cheetah_hip_model_set_unit": (_c.c_int, [_VP, _c.c_char_p, _VP, _SZ, _c.c_uint32,
                                              _c.POINTER(_c.c_uint64), _SZ]),
    "cheetah_hip_model_finalize": (_c.c_int, [_VP]),
    "cheetah_hip_forward": (_c.c_int, [_VP, _U32P, _SZ, _SZ, _SZ, _F32P]),
    "cheetah_hip_forward_greedy": (_c.c_int, [_VP, _U32P, _SZ, _SZ, _SZ, _U32P, _F32P]),
    "cheetah_hip_decode_greedy": (_c.c_int, [_VP, _c.c_uint32, _SZ, _SZ, _U32P]),
    "cheetah_hip_clear_cache": (None, [_VP]),
    "cheetah_hip_clone": (_VP, [_VP]),
    "cheetah_hip_kv_len": (_SZ, [_VP]),
    "cheetah_hip_kv_snapshot": (_c.c_int, [_VP, _c.POINTER(_VP), _c.POINTER(_SZ)]),
    "cheetah_hip_restore_kv_prefix": (_c.c_int, [_VP, _VP, _SZ]),
    "cheetah_hip_snapshot_free": (None, [_VP]),
    "cheetah_hip_kv_download": (_c.c_int, [_VP, _c.c_uint32, _SZ, _SZ, _F32P, _F32P]),
    "cheetah_hip_model_free": (None, [_VP]),
    "cheetah_hip_evict_unit": (_c.c_int, [_VP, _c.c_char_p]),
    "cheetah_hip_page_in_unit": (_c.c_int, [_VP, _c.c_char_p, _c.c_int32]),
    "cheetah_hip_unit_tier": (_c.c_int, [_VP, _c.c_char_p]),
    "cheetah_hip_time_gemv": (_c.c_int, [_c.c_uint32, _c.POINTER(_VP), _SZ, _SZ, _SZ, _VP, _VP, _SZ, _F32P]),
    "cheetah_hip_time_decode": (_c.c_int, [_VP, _c.c_uint32, _SZ, _SZ, _F32P, _F32P, _U32P]),
    "cheetah_hip_time_gemm": (_c.c_int, [_c.c_uint32, _c.POINTER(_VP), _SZ, _SZ, _SZ, _VP, _SZ, _VP, _SZ, _F32P]),
    "cheetah_hip_time_attention": (_c.c_int, [_VP, _c.POINTER(KvView), _SZ, _c.c_uint32, _SZ, _SZ, _VP, _SZ,
                                               _F32P]),
}

_lib = None
_lock = threading.RLock()
_initialized = False


def lib():
    """Loads the library (no GPU call). Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                           "(make -C cheetah_amd/csrc). There is no CPU fallback.")
        L = _c.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _err() -> str:
    return lib().cheetah_hip_last_error().decode()


def check(rc: int) -> None:
    if rc != 0:
        raise HipError(_err())


def init(device: int = 0) -> None:
    global _initialized
    with _lock:
        if not _initialized:
            check(lib().cheetah_hip_init(device))
            _initialized = True


def device_name() -> str:
    return lib().cheetah_hip_device_name().decode()


def synchronize() -> None:
    check(lib().cheetah_hip_synchronize())


def copy(dst: "DeviceBuffer", src: "DeviceBuffer", nbytes: int) -> None:
    """Device-to-device copy of nbytes (cheetah_hip_copy)."""
    if nbytes > min(dst.nbytes, src.nbytes):
        raise ValueError("copy larger than a buffer")
    check(lib().cheetah_hip_copy(dst.ptr, src.ptr, int(nbytes)))


class DeviceBuffer:
    """A device allocation (cheetah_hip_alloc) with host copy helpers."""

    def __init__(self, nbytes: int):
        init()
        self.nbytes = int(nbytes)
        self.ptr = lib().cheetah_hip_alloc(self.nbytes)
        if not self.ptr:
            raise HipError(_err())

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(max(arr.nbytes, 1))
        if arr.nbytes:
            check(lib().cheetah_hip_upload(buf.ptr, arr.ctypes.data, arr.nbytes))
        return buf

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(lib().cheetah_hip_upload(self.ptr, arr.ctypes.data, arr.nbytes))

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        check(lib().cheetah_hip_download(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr and _lib is not None:
            _lib.cheetah_hip_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Op-level helpers (host arrays in, host arrays out).
# ---------------------------------------------------------------------------

def _fmt_name(fmt: str) -> str:
    if fmt not in ("bf16", "q8", "q4"):
        raise ValueError(f"unknown weight format {fmt!r}")
    return fmt


def buffer_bytes(fmt: str, rows: int, cols: int) -> int:
    if fmt == "bf16":
        return rows * cols * 2
    fn = lib().cheetah_hip_q8_buffer_bytes if fmt == "q8" else lib().cheetah_hip_q4_buffer_bytes
    return fn(rows, cols)


def gemv(w_dev: DeviceBuffer, fmt: str, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    if x.size != cols:
        raise ValueError("gemv input width mismatch")
    xd = DeviceBuffer.from_array(x)
    yd = DeviceBuffer(rows * 4)
    fn = getattr(lib(), f"cheetah_hip_gemv_{_fmt_name(fmt)}")
    check(fn(w_dev.ptr, rows, cols, xd.ptr, yd.ptr))
    return yd.download(np.float32, rows)


def gemm(w_dev: DeviceBuffer, fmt: str, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    n = x.shape[0]
    xd = DeviceBuffer.from_array(x)
    yd = DeviceBuffer(n * rows * 4)
    fn = getattr(lib(), f"cheetah_hip_gemm_{_fmt_name(fmt)}")
    check(fn(w_dev.ptr, rows, cols, xd.ptr, n, yd.ptr))
    return yd.download(np.float32, n * rows).reshape(n, rows)


def quantize(w_bf16: np.ndarray, fmt: str) -> np.ndarray:
    rows, cols = w_bf16.shape
    wd = DeviceBuffer.from_array(np.ascontiguousarray(w_bf16, np.uint16))
    size = buffer_bytes(fmt, rows, cols)
    od = DeviceBuffer(size)
    fn = getattr(lib(), f"cheetah_hip_quantize_{fmt}")
    check(fn(wd.ptr, rows, cols, od.ptr, size))
    return od.download(np.uint8, size)


def dequant(buf: np.ndarray, fmt: str, rows: int, cols: int) -> np.ndarray:
    bd = DeviceBuffer.from_array(np.ascontiguousarray(buf, np.uint8))
    od = DeviceBuffer(rows * cols * 4)
    fn = getattr(lib(), f"cheetah_hip_dequant_{fmt}")
    check(fn(bd.ptr, rows, cols, od.ptr))
    return od.download(np.float32, rows * cols).reshape(rows, cols)


def paged_kv(keys_bf16: np.ndarray, values_bf16: np.ndarray, page_size: int = 64, seed: int = 0):
    """Lays [ctx, kv_heads, head_dim] BF16 K/V out as shuffled pages
    [page][kv_head][page_size][head_dim] plus a page table."""
    ctx, kvh, hd = keys_bf16.shape
    npages = (ctx + page_size - 1) // page_size
    perm = np.random.default_rng(seed).permutation(npages).astype(np.int32)
    kp = np.zeros((npages, kvh, page_size, hd), np.uint16)
    vp = np.zeros_like(kp)
    for lp in range(npages):
        seg = slice(lp * page_size, min(ctx, (lp + 1) * page_size))
        n = seg.stop - seg.start
        kp[perm[lp], :, :n] = keys_bf16[seg].transpose(1, 0, 2)
        vp[perm[lp], :, :n] = values_bf16[seg].transpose(1, 0, 2)
    return kp, vp, perm


def attention(q: np.ndarray, kp: np.ndarray, vp: np.ndarray, table: np.ndarray, q_heads: int, rows: int,
              offset: int, noalloc: bool = False) -> np.ndarray:
    """q: f32 [rows, q_heads*hd]; kp/vp: BF16 pages; table: int32 page table.
    noalloc: through cheetah_hip_attention_noalloc (fixed device scratch)."""
    _, kvh, ps, hd = kp.shape
    qd = DeviceBuffer.from_array(np.ascontiguousarray(q, np.float32))
    kd, vd, td = DeviceBuffer.from_array(kp), DeviceBuffer.from_array(vp), DeviceBuffer.from_array(table)
    od = DeviceBuffer(rows * q_heads * hd * 4)
    view = KvView(kd.ptr, vd.ptr, td.ptr, ps, kvh, hd)
    fn = lib().cheetah_hip_attention_noalloc if noalloc else lib().cheetah_hip_attention
    check(fn(qd.ptr, _c.byref(view), q_heads, rows, offset, od.ptr))
    return od.download(np.float32, rows * q_heads * hd).reshape(rows, q_heads * hd)


# ---------------------------------------------------------------------------
# The model: HIP implementation of ModelForward (registry.rs:57-85).
# ---------------------------------------------------------------------------

def make_config(shape) -> Config:
    return Config(shape.family, shape.num_layers, shape.hidden_size, shape.q_heads, shape.kv_heads,
                  shape.head_dim, shape.rotary_dim, shape.intermediate_size, shape.vocab_size,
                  int(shape.tie_word_embeddings), shape.sliding_window, shape.rope_theta, shape.rms_eps)


class Snapshot:
    def __init__(self, handle, positions: int):
        self._h = handle
        self.positions = positions

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.cheetah_hip_snapshot_free(self._h)
            self._h = None


class HipForward:
    """forward / clear_cache / kv_snapshot / restore_kv_prefix / device_name /
    clone, with the ModelForward semantics (registry.rs:57-85)."""

    def __init__(self, shape, weights: dict | None = None, quant=None, kv_capacity: int = 0,
                 max_chunk_rows: int = 0, kv: str = "bf16", _handle=None):
        init()
        self.shape = shape
        L = lib()
        if _handle is not None:
            self._h = _handle
            return
        if kv not in KV_FORMATS:
            raise ValueError(f"kv must be one of {sorted(KV_FORMATS)}")
        cfg = make_config(shape)
        h = L.cheetah_hip_model_create(_c.byref(cfg), QUANT[quant], KV_FORMATS[kv], kv_capacity, max_chunk_rows)
        if not h:
            raise HipError(_err())
        self._h = h
        for name, arr in (weights or {}).items():
            self.set_unit(name, arr)
        if weights is not None:
            self.finalize()

    def set_unit(self, name: str, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.dtype != np.uint16:
            raise HipError(f"HIP backend: unit '{name}' is not BF16 (the served stored precision).")
        dims = (_c.c_uint64 * arr.ndim)(*arr.shape)
        check(lib().cheetah_hip_model_set_unit(self._h, name.encode(), arr.ctypes.data, arr.nbytes, 1, dims,
                                               arr.ndim))

    def finalize(self) -> None:
        check(lib().cheetah_hip_model_finalize(self._h))

    def forward(self, tokens, offset: int, chunk_rows: int = 0) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.shape.vocab_size, np.float32)
        check(lib().cheetah_hip_forward(self._h, toks.ctypes.data_as(_U32P), toks.size, offset, chunk_rows,
                                        logits.ctypes.data_as(_F32P)))
        return logits

    def forward_greedy(self, tokens, offset: int, chunk_rows: int = 0, want_logits: bool = False):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = _c.c_uint32(0)
        logits = np.empty(self.shape.vocab_size, np.float32) if want_logits else None
        check(lib().cheetah_hip_forward_greedy(self._h, toks.ctypes.data_as(_U32P), toks.size, offset, chunk_rows,
                                               _c.byref(nxt),
                                               logits.ctypes.data_as(_F32P) if want_logits else None))
        return (int(nxt.value), logits) if want_logits else int(nxt.value)

    def decode_greedy(self, token: int, offset: int, steps: int) -> np.ndarray:
        out = np.zeros(steps, np.uint32)
        check(lib().cheetah_hip_decode_greedy(self._h, int(token), offset, steps, out.ctypes.data_as(_U32P)))
        return out

    def time_decode(self, token: int, offset: int, steps: int):
        ms = _c.c_float(0)
        gms = _c.c_float(0)
        out = np.zeros(steps, np.uint32)
        check(lib().cheetah_hip_time_decode(self._h, int(token), offset, steps, _c.byref(ms), _c.byref(gms),
                                            out.ctypes.data_as(_U32P)))
        return ms.value, gms.value, out

    def clear_cache(self) -> None:
        lib().cheetah_hip_clear_cache(self._h)

    def device_name(self) -> str:
        return device_name()

    def kv_len(self) -> int:
        return lib().cheetah_hip_kv_len(self._h)

    def clone(self) -> "HipForward":
        h = lib().cheetah_hip_clone(self._h)
        if not h:
            raise HipError(_err())
        return HipForward(self.shape, _handle=h)

    def kv_snapshot(self) -> Snapshot:
        h = _VP()
        pos = _SZ(0)
        check(lib().cheetah_hip_kv_snapshot(self._h, _c.byref(h), _c.byref(pos)))
        return Snapshot(h, pos.value)

    def restore_kv_prefix(self, snapshot: Snapshot, positions: int) -> bool:
        check(lib().cheetah_hip_restore_kv_prefix(self._h, snapshot._h, positions))
        return True

    def kv_rows(self, layer: int, pos_begin: int, n: int):
        """Cached K and V of positions [pos_begin, pos_begin + n) of one
        layer as f32 [n, kv_heads, head_dim] (the reference's cache rows)."""
        shp = (n, self.shape.kv_heads, self.shape.head_dim)
        k = np.empty(shp, np.float32)
        v = np.empty(shp, np.float32)
        check(lib().cheetah_hip_kv_download(self._h, layer, pos_begin, n, k.ctypes.data_as(_F32P),
                                            v.ctypes.data_as(_F32P)))
        return k, v

    def page_in_unit(self, unit_id: str, tier: int = 0) -> bool:
        """AntTierControl::page_in_unit (registry.rs:89): moves a per-layer
        linear weight back into HBM; True when the id names one (tier is
        ignored, as every reference implementation ignores it)."""
        rc = lib().cheetah_hip_page_in_unit(self._h, unit_id.encode(), int(tier))
        if rc < 0:
            raise HipError(_err())
        return rc == 1

    def evict_unit(self, unit_id: str) -> bool:
        """AntTierControl::evict_unit (registry.rs:91): releases a per-layer
        linear weight's HBM buffer, keeping a pinned host copy that forwards
        stream one layer ahead; True when the id names one."""
        rc = lib().cheetah_hip_evict_unit(self._h, unit_id.encode())
        if rc < 0:
            raise HipError(_err())
        return rc == 1

    def unit_tier(self, unit_id: str) -> int:
        """1 = HBM, 2 = pinned host memory, 0 = not a movable unit."""
        rc = lib().cheetah_hip_unit_tier(self._h, unit_id.encode())
        if rc < 0:
            raise HipError(_err())
        return rc

    def close(self) -> None:
        if getattr(self, "_h", None) and _lib is not None:
            _lib.cheetah_hip_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()
