"""Op-level measurements on one GPU: the attention op and the quantized
GEMV/GEMM at the shapes the decoder path runs (32 q / 8 KV heads of 128;
4096x4096, 4096x14336, 14336x4096 in the Q8/Q4 layouts of
src/chat/precision/q8.rs and q4.rs).

Every timing rotates over device buffers whose total exceeds the 256 MB
Infinity Cache, so each launch streams from HBM, and uses HIP events on the
stream the kernels run on.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip

HBM_PEAK_GBPS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 640 << 20

FMT_CODE = {"bf16": 1, "q8": 4, "q4": 5}


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    return (_bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def _replicas(host: np.ndarray, count: int) -> list:
    """`count` device copies of one host buffer (one upload, device copies)."""
    first = hip.DeviceBuffer.from_array(host)
    bufs = [first]
    for _ in range(count - 1):
        b = hip.DeviceBuffer(host.nbytes)
        hip.copy(b, first, host.nbytes)
        bufs.append(b)
    return bufs


def quantized_weights(fmt: str, rows: int, cols: int, seed: int) -> np.ndarray:
    """A buffer in the reference layout: f32 scales uniform in [1e-3, 1e-2],
    codes uniform over the format's range (Q8 [-127, 127], Q4 [-8, 7]); BF16:
    normal(0, 0.02) rounded to BF16 (the synthetic model weights)."""
    rng = np.random.default_rng(seed)
    if fmt == "bf16":
        return _bf16_bits((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)).view(np.uint8).reshape(-1)
    total = hip.buffer_bytes(fmt, rows, cols)
    stride = (total - rows * 4) // rows
    out = np.zeros(total, np.uint8)
    out[: rows * 4] = rng.uniform(1e-3, 1e-2, rows).astype(np.float32).view(np.uint8)
    body = out[rows * 4:].reshape(rows, stride)
    if fmt == "q8":
        body[:, :cols] = rng.integers(-127, 128, (rows, cols)).astype(np.int8).view(np.uint8)
    else:
        codes = rng.integers(-8, 8, (rows, cols)).astype(np.int16) & 0xF
        if cols % 2:
            codes = np.concatenate([codes, np.zeros((rows, 1), np.int16)], axis=1)
        packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
        body[:, : packed.shape[1]] = packed
    return out


def gemv_gemm(shapes=((4096, 4096), (4096, 14336), (14336, 4096)), fmts=("q8", "q4"), iters: int = 20,
              gemm_n: int = 512, gemm_iters: int = 3) -> list:
    lib = hip.lib()
    rng = np.random.default_rng(7)
    out = []
    for fmt in fmts:
        for rows, cols in shapes:
            host = quantized_weights(fmt, rows, cols, seed=rows * 31 + cols)
            nbuf = max(2, -(-ROTATE_BYTES // host.nbytes))
            bufs = _replicas(host, nbuf)
            ptrs = (ctypes.c_void_p * nbuf)(*[b.ptr for b in bufs])
            x = _bf16_round(rng.standard_normal(cols).astype(np.float32))
            xd = hip.DeviceBuffer.from_array(x)
            yd = hip.DeviceBuffer(rows * 4)
            ms = ctypes.c_float()
            hip.check(lib.cheetah_hip_time_gemv(FMT_CODE[fmt], ptrs, nbuf, rows, cols, xd.ptr, yd.ptr, iters,
                                                ctypes.byref(ms)))
            gemv_bytes = host.nbytes + cols * 4 + rows * 4
            xs = _bf16_round(rng.standard_normal((gemm_n, cols)).astype(np.float32))
            xsd = hip.DeviceBuffer.from_array(xs)
            ysd = hip.DeviceBuffer(gemm_n * rows * 4)
            gms = ctypes.c_float()
            hip.check(lib.cheetah_hip_time_gemm(FMT_CODE[fmt], ptrs, min(nbuf, 4), rows, cols, xsd.ptr, gemm_n,
                                                ysd.ptr, gemm_iters, ctypes.byref(gms)))
            flops = 2.0 * gemm_n * rows * cols
            out.append({
                "fmt": fmt, "rows": rows, "cols": cols, "buffer_bytes": host.nbytes, "rotating_buffers": nbuf,
                "gemv_ms": round(ms.value, 5),
                "gemv_gbps": round(gemv_bytes / (ms.value * 1e-3) / 1e9, 1),
                "gemv_hbm_frac": round(gemv_bytes / (ms.value * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                f"gemm_n{gemm_n}_ms": round(gms.value, 4),
                f"gemm_n{gemm_n}_tflops": round(flops / (gms.value * 1e-3) / 1e12, 2),
                f"gemm_n{gemm_n}_mfma_frac": round(flops / (gms.value * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 5),
            })
            for b in bufs + [xd, yd, xsd, ysd]:
                b.free()
    return out


def attention(lengths=(1024, 4096, 16384), nbuf: int = 8, iters: int = 40, prefill_rows: int = 512,
              prefill_offset: int = 4096, prefill_iters: int = 3) -> dict:
    """GQA 32q/8kv/128 over BF16 paged KV: decode (one query row at context
    L) and one prefill chunk (512 rows appended to a 4096-position prefix,
    causal)."""
    lib = hip.lib()
    q_heads, kv_heads, hd, page = 32, 8, 128, 64
    max_ctx = max(max(lengths), prefill_offset + prefill_rows)
    pages = -(-max_ctx // page)
    rng = np.random.default_rng(11)
    pool = rng.standard_normal((pages, kv_heads, page, hd)).astype(np.float32)
    kbits = _bf16_bits(pool)
    vbits = _bf16_bits(rng.standard_normal((pages, kv_heads, page, hd)).astype(np.float32))
    kbufs, vbufs = _replicas(kbits, nbuf), _replicas(vbits, nbuf)
    table = hip.DeviceBuffer.from_array(np.arange(pages, dtype=np.int32))
    views = (hip.KvView * nbuf)(*[hip.KvView(kbufs[i].ptr, vbufs[i].ptr, table.ptr, page, kv_heads, hd)
                                  for i in range(nbuf)])
    res = {"heads": "32 q / 8 KV, head_dim 128, BF16 KV pages of 64", "rotating_caches": nbuf,
           "cache_bytes_each": int(kbits.nbytes * 2), "decode": []}
    qd = hip.DeviceBuffer.from_array(rng.standard_normal(q_heads * hd).astype(np.float32))
    od = hip.DeviceBuffer(q_heads * hd * 4)
    for L in lengths:
        ms = ctypes.c_float()
        hip.check(lib.cheetah_hip_time_attention(qd.ptr, views, nbuf, q_heads, 1, L - 1, od.ptr, iters,
                                                 ctypes.byref(ms)))
        nbytes = 4096 * L + 16384
        res["decode"].append({"context": L, "ms": round(ms.value, 5), "bytes": nbytes,
                              "gbps": round(nbytes / (ms.value * 1e-3) / 1e9, 1),
                              "hbm_frac": round(nbytes / (ms.value * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)})
    qp = hip.DeviceBuffer.from_array(rng.standard_normal((prefill_rows, q_heads * hd)).astype(np.float32))
    op = hip.DeviceBuffer(prefill_rows * q_heads * hd * 4)
    ms = ctypes.c_float()
    hip.check(lib.cheetah_hip_time_attention(qp.ptr, views, nbuf, q_heads, prefill_rows, prefill_offset, op.ptr,
                                             prefill_iters, ctypes.byref(ms)))
    flops = 4.0 * q_heads * hd * sum(prefill_offset + 1 + i for i in range(prefill_rows))
    res["prefill_chunk"] = {"rows": prefill_rows, "prefix": prefill_offset, "ms": round(ms.value, 4),
                            "flops": flops, "tflops": round(flops / (ms.value * 1e-3) / 1e12, 2),
                            "mfma_frac": round(flops / (ms.value * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 5)}
    for b in kbufs + vbufs + [table, qd, od, qp, op]:
        b.free()
    return res


def main(argv=None) -> int:
    """python -m cheetah_amd.opbench [attention] [gemv] [gemm]: one JSON line
    per measurement (all three when no part is named)."""
    import argparse
    import json

    ap = argparse.ArgumentParser()
    ap.add_argument("parts", nargs="*", help="attention, gemv and/or gemm")
    ap.add_argument("--shapes", default="4096x4096,4096x14336,14336x4096")
    ap.add_argument("--fmts", default="q8,q4")
    args = ap.parse_args(argv)
    parts = set(args.parts or ["attention", "gemv", "gemm"])
    if parts - {"attention", "gemv", "gemm"}:
        ap.error(f"unknown part(s): {sorted(parts - {'attention', 'gemv', 'gemm'})}")
    hip.init(0)
    if "attention" in parts:
        print(json.dumps({"attention": attention()}), flush=True)
    if parts & {"gemv", "gemm"}:
        shapes = tuple(tuple(int(v) for v in s.split("x")) for s in args.shapes.split(","))
        for r in gemv_gemm(shapes=shapes, fmts=tuple(args.fmts.split(",")),
                           gemm_iters=3 if "gemm" in parts else 1):
            if "gemm" not in parts:
                r = {k: v for k, v in r.items() if not k.startswith("gemm")}
            print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
