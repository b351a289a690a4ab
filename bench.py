#!/usr/bin/env python3
"""Decoder-forward benchmark on one MI355X.

Workload (one "step"): the Qwen2-0.5B-architecture decoder with seeded
random-init BF16 weights serves one generation at batch 1 — a 512-token
seeded prompt prefilled in chunks of 128 through the HIP ModelForward, then
128 greedy decode steps (the Engine::generate_inner loop, engine.rs:1837-1979,
with argmax on the device). `value` is decode tokens/s of the whole job;
prefill tokens/s, the decode step's effective HBM rate and the dominant
kernel's roofline are reported beside it, with the CPU oracle (a C++
restatement of the reference's native AVX2 backend) timed on this host.

Beside it: the same generation through the per-step ModelForward::forward
path (logits to the host), with the reference's f32 KV cache, the greedy
ids against the oracle's goldens (BF16-KV run and reference semantics), the
Llama-3-8B Q4 (8K prompt) and Qwen2-7B (32K prompt, prefix reuse) decoders
as `large`, and the op-level attention / GEMV / GEMM figures as `ops`.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s & prefill tok/s (1 GPU); attention+GEMV HBM GB/s vs peak"
HBM_PEAK_GBPS = 8000.0
PROMPT = 512
CHUNK = 128
DECODE = 128


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_cpus():
    """The host cores this process may run on: the CPU model, the logical
    CPUs in its affinity mask and the physical cores they belong to (sysfs
    core_id per package). The reference sizes its pool to physical cores
    (num_cpus::get_physical, engine.rs:859)."""
    logical = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores = set()
    for c in logical:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "logical_cpus": len(logical), "physical_cores": len(cores),
            "machine_logical_cpus": os.cpu_count()}


def cpu_baseline(shape, weights, prompt, decode_steps: int):
    """The CPU oracle on a bounded sample of the same workload: the full
    512-token prefill (128-row chunks) and `decode_steps` greedy decodes, on
    a pool of one thread per physical core this process may use."""
    from cheetah_amd import workloads
    from oracle import oracle

    cpus = host_cpus()
    threads = max(1, cpus["physical_cores"])
    oracle.set_threads(threads)
    m = oracle.RefModel(shape, weights)
    t0 = time.perf_counter()
    logits = m.forward(prompt, 0, chunk_rows=CHUNK)
    t1 = time.perf_counter()
    for step in range(decode_steps):
        tok = workloads.greedy_token(logits)
        logits = m.forward([tok], PROMPT + step)
    t2 = time.perf_counter()
    return {
        "value": round(decode_steps / (t2 - t1), 3),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"decode tok/s over {decode_steps} greedy steps after the full {PROMPT}-token prefill "
                  f"(prefill {PROMPT / (t1 - t0):.1f} tok/s); C++ restatement of the reference native "
                  f"AVX2 path, one thread per physical core ({threads})",
        "prefill_tok_s": round(PROMPT / (t1 - t0), 3),
        "threads": threads,
        "cores_physical": cpus["physical_cores"],
        "logical_cpus": cpus["logical_cpus"],
        "machine_logical_cpus": cpus["machine_logical_cpus"],
        "cpu_model": cpus["cpu_model"],
    }


def host_tier(g, shape, prompt, resident_tokens, decode_steps: int = 32):
    """One generation with every layer's linear weights evicted to pinned
    host memory (Ant tier control, engine.rs:1210-1226): each forward streams
    all layers' matrices over PCIe into the feed slots, so this is the
    host-to-device copy rate, not an HBM figure. Pages everything back in."""
    names = ["self_attn.q_proj", "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    units = [f"model.layers.{l}.{n}.weight" for l in range(shape.num_layers) for n in names]
    for u in units:
        assert g.evict_unit(u), u
    g.clear_cache()
    t0 = time.perf_counter()
    first = g.forward_greedy(prompt, 0, chunk_rows=CHUNK)
    t1 = time.perf_counter()
    rest = g.decode_greedy(first, len(prompt), decode_steps)
    t2 = time.perf_counter()
    toks = [first] + rest.tolist()
    for u in units:
        assert g.page_in_unit(u, 0), u
    streamed = shape.linear_params() * 2  # BF16 bytes of every layer's matrices
    dec_s = (t2 - t1) / decode_steps
    return {
        "layers_on_host": shape.num_layers,
        "streamed_bytes_per_forward": streamed,
        "decode_tok_s": round(1.0 / dec_s, 2),
        "prefill_tok_s": round(len(prompt) / (t1 - t0), 1),
        "h2d_gbps_decode": round(streamed / dec_s / 1e9, 1),
        "tokens_match_resident": toks == resident_tokens[:decode_steps + 1],
    }


def _golden(name):
    path = os.path.join(ROOT, "tests", "golden", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


LARGE = {
    "llama3-8b-q4": ("llama3-8b architecture (32 layers, hidden 4096, 32/8 heads, hd 128, ffn 14336, vocab 128256), "
                     "Q4 linears quantized on the device from seeded BF16 weights, BF16 head, BF16 paged KV; "
                     "8192-token prompt in 512-row chunks, then 256 greedy decode steps, batch 1"),
    "qwen2-7b-32k": ("qwen2-7b architecture (28 layers, hidden 3584, 28/4 heads, hd 128, ffn 18944, vocab 152064), "
                     "BF16 weights and paged KV; turn 1: 32768-token prompt in 1024-row chunks + KV snapshot; "
                     "turn 2: restore 30720 positions, 2048-token suffix in 1024-row chunks, 128 greedy decodes"),
}
MFMA_PEAK_TFLOPS = 2500.0


def _match32(tokens, gold):
    if gold is None:
        return None
    n = min(32, len(gold["tokens"]))
    return tokens[:n] == gold["tokens"][:n]


def measure_large(name: str) -> dict:
    """One timed pass of a large decoder (no warmup: each phase is long and
    the kernels are already built). Decode tok/s with the device's BF16 KV
    cache, prefill tok/s, their roofline fractions, and the greedy ids
    against the oracle's goldens: the BF16-KV run and the reference
    semantics (f32 KV)."""
    from cheetah_amd import configs, hip, workloads

    hip.init(0)
    if name == "llama3-8b-q4":
        shape = configs.LLAMA3_8B
        g, info = workloads.llama3_8b_q4(decode_steps=256)
        lin_bytes = sum(hip.buffer_bytes("q4", r, c) for layer in range(shape.num_layers)
                        for _, r, c in shape.linear_units(layer))
        weight_bytes = lin_bytes + shape.head_params() * 2
        ctx_mid = 8192 + 128
        pre_flops = sum(workloads.prefill_flops(shape, 512, off) for off in range(0, 8192, 512))
        pre_s = info["prefill_s"]
        gold_bf16 = _golden("llama3_8b_q4_bf16kv_greedy.json")
        gold_ref = _golden("llama3_8b_q4_greedy.json")
        extra = {"prefill_tok_s": info["prefill_tok_s"]}
    else:
        shape = configs.QWEN2_7B
        g, info = workloads.qwen2_7b_32k(decode_steps=128)
        weight_bytes = (shape.linear_params() + shape.head_params()) * 2
        ctx_mid = 32768 + 64
        pre_flops = sum(workloads.prefill_flops(shape, 1024, off) for off in range(0, 32768, 1024))
        pre_s = info["turn1_prefill_s"]
        gold_bf16 = _golden("qwen2_7b_32k_greedy.json")
        gold_ref = _golden("qwen2_7b_32k_f32kv_greedy.json")
        extra = {"prefill_tok_s": info["turn1_prefill_tok_s"], "turn2_prefill_tok_s": info["turn2_prefill_tok_s"],
                 "snapshot_s": info["snapshot_s"], "restore_s": info["restore_s"]}
    g.close()
    step_bytes = workloads.decode_bytes(shape, ctx_mid, weight_bytes)
    ms_tok = 1e3 / info["decode_tok_s"]
    gbps = step_bytes / (ms_tok * 1e-3) / 1e9
    tflops = pre_flops / pre_s / 1e12
    return {
        "workload": LARGE[name],
        "decode_tok_s": info["decode_tok_s"],
        **extra,
        "wall_ms": round((info.get("prefill_s", 0) + info.get("turn1_prefill_s", 0) + info.get("turn2_prefill_s", 0)
                          + info["decode_s"]) * 1e3, 3),
        "decode_ms_per_token": round(ms_tok, 4),
        "decode_effective_gbps": round(gbps, 1), "decode_hbm_roofline_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "decode_bytes_per_token": int(step_bytes),
        "prefill_tflops": round(tflops, 2), "prefill_mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
        "prefill_flops": pre_flops,
        "kv_cache": "bf16",
        "greedy_first32_match_bf16kv_oracle": _match32(info["tokens"], gold_bf16),
        "greedy_first32_match_reference": _match32(info["tokens"], gold_ref),
        "load": {"synth_s": info.get("synth_s"), "upload_s": info.get("upload_s")},
    }


def large_workload(args) -> int:
    """The large decoder's own line: decode tok/s is `value`."""
    r = measure_large(args.workload)
    result = {
        "metric": METRIC, "value": r["decode_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": 1, "warmup": 0,
        "ms_per_step": r["wall_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4 weights, bf16 activations" if args.workload == "llama3-8b-q4" else "bf16",
        "data": "synthetic: seeded random-init weights (normal 0.02), seeded uniform token ids",
        "config": {"workload": r["workload"], "global_batch": 1, "parallelism": "none (1 GPU)"},
        **{k: v for k, v in r.items() if k not in ("workload", "decode_tok_s", "wall_ms")},
    }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cpu-decode-steps", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-residency", action="store_true",
                    help="skip the host-tier (evicted weights) generation")
    ap.add_argument("--no-ops", action="store_true",
                    help="skip the op-level attention / GEMV / GEMM measurements")
    ap.add_argument("--no-large", action="store_true",
                    help="skip the Llama-3-8B Q4 and Qwen2-7B 32K sub-measurements")
    ap.add_argument("--workload", default="qwen2-0.5b", choices=["qwen2-0.5b", "llama3-8b-q4", "qwen2-7b-32k"],
                    help="qwen2-0.5b (the headline line); the two large decoders print their own line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device-to-device 3 times (calibrates rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        from cheetah_amd import hip

        src, dst = hip.DeviceBuffer(1 << 30), hip.DeviceBuffer(1 << 30)
        for _ in range(3):
            hip.copy(dst, src, 1 << 30)
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "copies": 3}))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported "
                                   "(the decoder is not sharded)", "n_gpus": args.gpus}))
        return 2

    if args.workload != "qwen2-0.5b":
        return large_workload(args)

    import numpy as np

    from cheetah_amd import configs, hip, synth, workloads

    shape = configs.QWEN2_0_5B
    hip.init(0)
    log(f"[bench] device {hip.device_name()}")
    t = time.perf_counter()
    weights = synth.make_weights(shape)
    log(f"[bench] weights synthesized in {time.perf_counter() - t:.1f}s")
    t = time.perf_counter()
    g = hip.HipForward(shape, weights, kv_capacity=2048, max_chunk_rows=CHUNK)
    log(f"[bench] model uploaded in {time.perf_counter() - t:.1f}s")
    prompt = synth.make_tokens(shape.vocab_size, PROMPT, seed=1)

    def generation():
        g.clear_cache()
        t0 = time.perf_counter()
        first = g.forward_greedy(prompt, 0, chunk_rows=CHUNK)
        t1 = time.perf_counter()
        rest = g.decode_greedy(first, PROMPT, DECODE)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, [first] + rest.tolist()

    for i in range(args.warmup):
        generation()
        log(f"[bench] warmup {i + 1}/{args.warmup} done")
    hip.synchronize()
    T0 = time.perf_counter()
    pre, dec, tokens = 0.0, 0.0, None
    for i in range(args.steps):
        p, d, tokens = generation()
        pre += p
        dec += d
    hip.synchronize()
    T1 = time.perf_counter()
    log(f"[bench] timed {args.steps} generations in {T1 - T0:.3f}s")
    decode_tok_s = args.steps * DECODE / dec
    prefill_tok_s = args.steps * PROMPT / pre

    # The decode loop timed with HIP events on the model's stream: one launch
    # of the persistent decode kernel runs all DECODE steps (the dominant and
    # only kernel of the decode phase). Then the multi-kernel path's dominant
    # GEMV (gate/up with fused RMSNorm + SwiGLU) alone, cycling the layers.
    g.clear_cache()
    first = g.forward_greedy(prompt, 0, chunk_rows=CHUNK)
    ms_step, gemv_ms, _ = g.time_decode(first, PROMPT, DECODE)
    H, I = shape.hidden_size, shape.intermediate_size
    gemv_bytes = 2 * I * H * 2 + H * 4 + H * 2 + I * 4  # gate+up BF16, hidden, gain, out
    gemv_gbps = gemv_bytes / (gemv_ms * 1e-3) / 1e9
    # Algorithmic bytes of one decode step at context c: every weight once
    # (linear + tied head, BF16), the K/V rows of c positions read and one
    # position written (24 layers x K,V x 2 KV heads x 64 x 2 B = 12,288 B
    # per position).
    weight_bytes = (shape.linear_params() + shape.head_params()) * 2
    kv_pos_bytes = shape.num_layers * 2 * shape.kv_dim * 2
    ctx_sum = sum(p + 1 for p in range(PROMPT, PROMPT + DECODE))
    launch_bytes = DECODE * weight_bytes + kv_pos_bytes * (ctx_sum + DECODE)
    launch_ms = ms_step * DECODE
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    step_bytes = launch_bytes / DECODE
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_flow_qwen2_0_5b_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    gold_bf16 = _golden("qwen2_0_5b_bf16kv_greedy.json")
    gold_ref = _golden("qwen2_0_5b_greedy.json")
    departure = None
    if gold_ref is not None:
        departure = next((i for i in range(min(len(tokens), len(gold_ref["tokens"])))
                          if tokens[i] != gold_ref["tokens"][i]), None)

    # The ModelForward contract path: one cheetah_hip_forward per decode step
    # returning the vocabulary's logits to the host, greedy argmax on the host
    # (ties to the last index), as Engine::generate_inner samples
    # (engine.rs:1918-1935, 2247-2253).
    def per_step_generation():
        g.clear_cache()
        logits = g.forward(prompt, 0, chunk_rows=CHUNK)
        out = []
        t0 = time.perf_counter()
        for step in range(DECODE):
            tok = workloads.greedy_token(logits)
            out.append(tok)
            logits = g.forward(np.array([tok], np.uint32), PROMPT + step)
        return time.perf_counter() - t0, out

    per_step_generation()
    ps_s, ps_tokens = per_step_generation()
    log("[bench] per-step forward path timed")

    # The reference's own KV precision (f32 cache): decode rate and token
    # identity with the reference's greedy ids.
    g32 = hip.HipForward(shape, weights, kv_capacity=2048, max_chunk_rows=CHUNK, kv="f32")

    def generation32():
        g32.clear_cache()
        first = g32.forward_greedy(prompt, 0, chunk_rows=CHUNK)
        t1 = time.perf_counter()
        rest = g32.decode_greedy(first, PROMPT, DECODE)
        return time.perf_counter() - t1, [first] + rest.tolist()

    generation32()
    f32_s, f32_tokens = generation32()
    g32.close()
    log("[bench] f32-KV generation timed")

    result = {
        "metric": METRIC,
        "value": round(decode_tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((T1 - T0) / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded random-init BF16 weights (normal 0.02), seeded uniform token ids",
        "config": {
            "workload": "qwen2-0.5b architecture (24 layers, hidden 896, 14/2 heads, hd 64, ffn 4864, "
                        "vocab 151936), BF16 weights; 512-token prompt prefilled in 128-row chunks, then "
                        "128 greedy decode steps, batch 1",
            "global_batch": 1,
            "seq_len": PROMPT + DECODE,
            "parallelism": "none (1 GPU)",
        },
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_ms_per_token": round(dec / (args.steps * DECODE) * 1e3, 4),
        "decode_event_ms_per_token": round(ms_step, 4),
        "decode_effective_gbps": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "decode_hbm_roofline_frac": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "kv_cache": "bf16",
        "greedy_first32_match_bf16kv_oracle": _match32(tokens, gold_bf16),
        "greedy_first32_match_reference": _match32(tokens, gold_ref),
        "reference_departure": None if departure is None else {
            "step": departure, "reference_top2_margin": round(gold_ref["top2_margins"][departure], 5)},
        "f32_kv": {
            "decode_tok_s": round(DECODE / f32_s, 2),
            "greedy_first32_match_reference": _match32(f32_tokens, gold_ref),
        },
        "forward_per_step": {
            "path": "cheetah_hip_forward per decode step, logits to the host, host argmax (ModelForward::forward)",
            "decode_tok_s": round(DECODE / ps_s, 2),
            "tokens_match_device_greedy": ps_tokens == tokens[:DECODE],
        },
        "roofline": {
            "kernel": f"decode_flow_kernel (persistent decode: {DECODE} steps per launch, BF16 weights, "
                      "BF16 paged KV)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(launch_bytes),
            "avg_launch_ms": round(launch_ms, 3),
        },
        "graph_path_gemv": {
            "kernel": "gemv_kernel<BF16> gate/up + SwiGLU (fused RMSNorm), 4864x896 x2",
            "achieved_gbps": round(gemv_gbps, 1),
            "bytes_per_launch": gemv_bytes,
            "avg_launch_ms": round(gemv_ms, 5),
        },
    }
    if not args.no_residency:
        result["host_tier"] = host_tier(g, shape, prompt, tokens)
    if not args.no_large:
        g.close()
        result["large"] = {}
        for name in LARGE:
            log(f"[bench] {name} ...")
            result["large"][name.replace("-", "_")] = measure_large(name)
    if not args.no_ops:
        from cheetah_amd import opbench

        g.close()
        log("[bench] op-level attention ...")
        ops = {"attention": opbench.attention()}
        log("[bench] op-level GEMV / GEMM ...")
        ops["gemv_gemm"] = opbench.gemv_gemm()
        result["ops"] = ops
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(shape, weights, prompt, args.cpu_decode_steps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
