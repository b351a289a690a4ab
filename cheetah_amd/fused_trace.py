"""Per-phase timeline of one persistent decode step (decode_flow_kernel).

Usage: python -m cheetah_amd.fused_trace [--steps N] [--context C] [--raw PATH]

Runs the Qwen2-0.5B-shape BF16 decoder (seeded synthetic weights), prefills C
prompt tokens, then decodes N tokens in one persistent launch with
CHEETAH_HIP_FUSED_TRACE set: thread 0 of every block stamps the device wall
clock (100 MHz) at fixed points of the last step. Prints, per layer phase, when
its producers finished and when its consumers were released, as a markdown
report: the critical path of a layer split into hand-offs (last producer
store -> consumers' inputs staged) and phase compute.

Stamp slots per layer l (16 l + k): 0 layer start, 1 A.in (QKV input normed
and staged), 2 A.out (QKV rows stored), 3 B.in (attention item's q/K/V
staged), 4 scores, 5 softmax, 6 weighted V + partials stored, 7 B.out
(weight rows of C/D/E issued), 8 C.in (partials merged), 14 o_proj dot,
9 C.out (hid0 stored), 10 D.in, 11 D.out (down partials stored, next QKV rows issued),
12 E.in, 15 down dot, 13 E.out (hid1 stored). After the layers: 16 L head.in,
16 L + 1 head.out, 16 L + 2 token known.
"""
import argparse
import os
import tempfile

import numpy as np

from . import configs, hip, synth

KCW = 7      # compute waves per block (rows per block of o_proj/down, QKV pairs)
KWAVES = 8


def block_roles(shape, blocks: int, context: int, kv_bf16: bool = True):
    """Block index sets per role, as the launcher assigns them
    (decode_fused.hip launch_one / head_split)."""
    H, I, hd = shape.hidden_size, shape.intermediate_size, shape.head_dim
    qh, kvh = shape.q_heads, shape.kv_heads
    g = qh // kvh
    npairs = (qh + 2 * kvh) * hd // 2
    nhb = (H + KCW - 1) // KCW
    nab = (npairs + KCW - 1) // KCW
    a0 = nhb if nhb + nab <= blocks else blocks - nab
    row = hd * (2 if kv_bf16 else 4)
    ip = 128 if row <= 256 else 64
    S = (context + ip - 1) // ip
    hs = g > 1 and kvh * S * g <= blocks
    items = kvh * S * (g if hs else 1)
    b_items = set(range(blocks - items, blocks))
    a_set = set(range(a0, a0 + nab))
    return {
        "H": sorted(range(nhb)),
        "A": sorted(a_set - b_items),
        "AB": sorted(a_set & b_items),
        "B": sorted(b_items - a_set),
        "all": list(range(blocks)),
        "Aall": sorted(a_set),
        "Ball": sorted(b_items),
    }


def report(t: np.ndarray, roles: dict, layers: int) -> str:
    t = np.where(t == 0, np.nan, t.astype(np.float64))
    us = (t - np.nanmin(t[:, 0])) / 100.0

    def med(rg, slot):
        return float(np.nanmedian(us[roles[rg], slot]))

    def mx(rg, slot):
        return float(np.nanmax(us[roles[rg], slot]))

    segs = {k: [] for k in ("A dot + store", "hand-off A->B", "attention item", "hand-off B->C (+ merge)",
                             "o_proj dot + store", "hand-off C->D", "gate/up dot + store", "hand-off D->E",
                             "down dot + store", "hand-off E->A(next)")}
    for l in range(1, layers - 1):
        b, n = 16 * l, 16 * (l + 1)
        segs["A dot + store"].append(mx("Aall", b + 2) - med("Aall", b + 1))
        segs["hand-off A->B"].append(med("Ball", b + 3) - mx("Aall", b + 2))
        segs["attention item"].append(mx("Ball", b + 6) - med("Ball", b + 3))
        segs["hand-off B->C (+ merge)"].append(med("H", b + 8) - mx("Ball", b + 6))
        segs["o_proj dot + store"].append(mx("H", b + 9) - med("H", b + 8))
        segs["hand-off C->D"].append(med("all", b + 10) - mx("H", b + 9))
        segs["gate/up dot + store"].append(mx("all", b + 11) - med("all", b + 10))
        segs["hand-off D->E"].append(med("H", b + 12) - mx("all", b + 11))
        segs["down dot + store"].append(mx("H", b + 13) - med("H", b + 12))
        segs["hand-off E->A(next)"].append(med("Aall", n + 1) - mx("H", b + 13))
    span = [med("Aall", 16 * (l + 1) + 1) - med("Aall", 16 * l + 1) for l in range(1, layers - 1)]
    lines = [f"Layers 1..{layers - 2}: mean span {np.mean(span):.2f} us per layer (median A.in to the next layer's "
             f"A.in); head.in -> token {mx('all', 16 * layers + 2) - med('all', 16 * layers):.1f} us.", "",
             "| segment (critical path of a layer) | mean us | min | max |", "|---|---:|---:|---:|"]
    for k, v in segs.items():
        lines.append(f"| {k} | {np.mean(v):.2f} | {np.min(v):.2f} | {np.max(v):.2f} |")
    lines.append(f"| sum | {sum(np.mean(v) for v in segs.values()):.2f} | | |")
    lines += ["", "Per-role stamps of layer 12, us from the median A.in (median / max over the role's blocks):", ""]
    names = {0: "start", 1: "A.in", 2: "A.out", 3: "B.in", 4: "score", 5: "softmax", 6: "PV", 7: "B.out", 8: "C.in",
             14: "C.dot", 9: "C.out", 10: "D.in", 11: "D.out", 12: "E.in", 15: "E.dot", 13: "E.out"}
    l = min(12, layers - 2)
    ref = med("Aall", 16 * l + 1)
    lines += ["| role (blocks) | " + " | ".join(names.values()) + " |", "|---|" + "---:|" * len(names)]
    for rn in ("H", "A", "AB", "B"):
        rg = roles[rn]
        if not rg:
            continue
        cells = []
        for i in names:
            c = us[rg, 16 * l + i] - ref
            cells.append("" if np.all(np.isnan(c)) else f"{np.nanmedian(c):.1f}/{np.nanmax(c):.1f}")
        lines.append(f"| {rn} ({rg[0]}-{rg[-1]}) | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--context", type=int, default=512)
    ap.add_argument("--raw", default="", help="keep the raw stamp file here")
    args = ap.parse_args()
    hip.init(0)
    shape = configs.QWEN2_0_5B
    g = hip.HipForward(shape, synth.make_weights(shape), kv_capacity=args.context + args.steps + 64,
                       max_chunk_rows=128, kv="bf16")
    prompt = synth.make_tokens(shape.vocab_size, args.context, seed=1)
    first = g.forward_greedy(prompt, 0, chunk_rows=128)
    g.decode_greedy(first, args.context, args.steps)  # warm-up launch
    g.clear_cache()
    first = g.forward_greedy(prompt, 0, chunk_rows=128)
    path = args.raw or os.path.join(tempfile.mkdtemp(), "stamps.txt")
    os.environ["CHEETAH_HIP_FUSED_TRACE"] = path
    try:
        g.decode_greedy(first, args.context, args.steps)
    finally:
        del os.environ["CHEETAH_HIP_FUSED_TRACE"]
    t = np.loadtxt(path, dtype=np.float64)
    roles = block_roles(shape, t.shape[0], args.context + args.steps)
    print(f"# Persistent decode phase timeline: Qwen2-0.5B shape, BF16 KV, context {args.context}, step "
          f"{args.steps} of {args.steps}, {t.shape[0]} blocks\n")
    print(report(t, roles, shape.num_layers))


if __name__ == "__main__":
    main()
