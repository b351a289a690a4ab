"""Per-phase timeline of one persistent decode step (decode_flow_kernel).

Usage: python -m cheetah_amd.fused_trace [--steps N] [--context C] [--raw PATH]

Runs the Qwen2-0.5B-shape BF16 decoder (seeded synthetic weights), prefills C
prompt tokens, then decodes N tokens in one persistent launch with
CHEETAH_HIP_FUSED_TRACE set: thread 0 of every block stamps the device wall
clock (100 MHz) at fixed points of the last step. Prints, per layer phase, when
its producers finished and when its consumers were released, as a markdown
report: the critical path of a layer split into hand-offs (last producer
store -> consumers' inputs staged) and phase compute.

Stamp slots per layer l (16 l + k): 0 layer start, 1 P1.in (items' and KV
blocks' input normed and staged), 2 q.out (an item's q rotated), 3 the
waves' attention partials over the cached rows, 4 new row (the new K/V row
polled and scored), 5 partials merged, 6 P1.out (items: o_proj partials stored; KV blocks: K/V stored),
7 refill issued, 8 C.in (owners: item partials gathered), 9 C.out (hid0
stored), 10 D.in (FFN blocks: input normed), 11 gate/up + SwiGLU, 12 D.out
(down partials stored), 13 E.in (owners: down partials gathered), 14 E.out
(hid1 stored). After the layers: 16 L head.in, 16 L + 1 head.out, 16 L + 2
token known.
"""
import argparse
import os
import tempfile

import numpy as np

from . import configs, hip, synth

KWAVES = 8
KV_LDS_MAX = 64 * 1024
IP_MAX = 256
MAX_SPLITS = 16


def item_slots(q_heads: int, kv_heads: int) -> list:
    """The block slot (within a run's heads_padded blocks, slot j on XCD
    j % 8) of each q head, as decode_fused.hip's item_slots places them: the
    heads of one KV group on their own XCDs where the group count divides 8
    and the slots allow, else head h in slot h."""
    qp = (q_heads + 7) // 8 * 8
    G = q_heads // kv_heads if kv_heads else 0
    xpg = 8 // kv_heads if kv_heads and kv_heads <= 8 and 8 % kv_heads == 0 else 0
    if qp <= 64 and xpg and G * kv_heads == q_heads and (G + xpg - 1) // xpg <= qp // 8:
        return [(h % G // xpg) * 8 + (h // G) * xpg + h % G % xpg for h in range(q_heads)]
    return list(range(q_heads))


def block_roles(shape, blocks: int, context: int, ctx_end: int = 0, kv_bf16: bool = True):
    """Block index sets per role at a step of context `context` in a launch
    whose last step reaches `ctx_end`, as the launcher assigns them
    (decode_fused.hip geometry / launch_one)."""
    H, I, hd = shape.hidden_size, shape.intermediate_size, shape.head_dim
    qh, kvh = shape.q_heads, shape.kv_heads
    ctx_end = ctx_end or context
    nf = blocks * 5 // 8
    n32 = (I + 31) // 32  # FFN blocks of exactly 32 rows where they fit and cover the owners
    if H // 8 <= n32 <= nf:
        nf = n32
    f0 = blocks - nf
    nkv = (kvh * hd + KWAVES - 1) // KWAVES
    kv0 = f0 - nkv
    qp = (qh + 7) // 8 * 8  # item (split s, head h) at block s * qp + slot(h)
    s_cap = min(MAX_SPLITS, kv0 // qp)
    row = hd * (2 if kv_bf16 else 4)
    ip_max, ip = 0, 64
    while ip <= IP_MAX and 2 * ip * row <= KV_LDS_MAX:
        ip_max, ip = ip, ip * 2
    ip = 64
    while ip < ip_max and (ctx_end + ip - 1) // ip > s_cap:
        ip *= 2
    S = (context + ip - 1) // ip
    rb = (I + nf - 1) // nf
    nbd = (I + rb - 1) // rb
    no = H // 8
    slot = item_slots(qh, kvh)
    items = [sp * qp + slot[h] for sp in range(S) for h in range(qh)]
    return {
        "items": items,
        "last": [b for b in items if b // qp == S - 1],
        "kv": list(range(kv0, kv0 + nkv)),
        "p1": items + list(range(kv0, kv0 + nkv)),
        "ffn": list(range(f0, f0 + nbd)),
        "owners": list(range(f0, f0 + no)),
        "all": list(range(blocks)),
        "ip": ip,
    }


SEGMENTS = ("q dot", "cached rows (per-wave partials)", "new K/V row (last runs)", "merge of the partials", "o_proj partials",
            "hand-off items -> owners", "merge + residual", "hand-off owners -> FFN (+ norm)", "gate/up + SwiGLU",
            "down partials", "hand-off FFN -> owners", "sum + residual", "hand-off owners -> items (+ norm)")


def report(t: np.ndarray, roles: dict, layers: int) -> str:
    t = np.where(t == 0, np.nan, t.astype(np.float64))
    us = (t - np.nanmin(t[:, 0])) / 100.0

    def med(rg, slot):
        return float(np.nanmedian(us[roles[rg], slot]))

    def mx(rg, slot):
        return float(np.nanmax(us[roles[rg], slot]))

    segs = {k: [] for k in SEGMENTS}
    kv_dot = []
    for l in range(1, layers - 1):
        b, n = 16 * l, 16 * (l + 1)
        # Consecutive points of the layer's critical path: the segments tile
        # the span from the items' input to the next layer's.
        pts = [med("items", b + 1), mx("items", b + 2), mx("items", b + 3), mx("last", b + 4), mx("items", b + 5),
               mx("items", b + 6), med("owners", b + 8), mx("owners", b + 9), med("ffn", b + 10),
               mx("ffn", b + 11), mx("ffn", b + 12), med("owners", b + 13), mx("owners", b + 14),
               med("items", n + 1)]
        for name, a, z in zip(SEGMENTS, pts, pts[1:]):
            segs[name].append(z - a)
        kv_dot.append(mx("kv", b + 6) - med("kv", b + 1))
    span = [med("items", 16 * (l + 1) + 1) - med("items", 16 * l + 1) for l in range(1, layers - 1)]
    lines = [f"Layers 1..{layers - 2}: mean span {np.mean(span):.2f} us per layer (median item input to the next "
             f"layer's); head.in -> token {mx('all', 16 * layers + 2) - med('all', 16 * layers):.1f} us; KV blocks' "
             f"dot + K/V store (beside the path) {np.mean(kv_dot):.2f} us.", "",
             "| segment (critical path of a layer) | mean us | min | max |", "|---|---:|---:|---:|"]
    for k, v in segs.items():
        lines.append(f"| {k} | {np.mean(v):.2f} | {np.min(v):.2f} | {np.max(v):.2f} |")
    lines.append(f"| sum | {sum(np.mean(v) for v in segs.values()):.2f} | | |")
    lines += ["", "Per-role stamps of layer 12, us from the median item input (median / max over the role's "
              "blocks):", ""]
    names = {0: "start", 1: "P1.in", 2: "q", 3: "scores", 4: "new row", 5: "PV", 6: "P1.out", 7: "refill",
             8: "C.in", 9: "C.out", 10: "D.in", 11: "gate/up", 12: "D.out", 13: "E.in", 14: "E.out"}
    l = min(12, layers - 2)
    ref = med("items", 16 * l + 1)
    lines += ["| role (blocks) | " + " | ".join(names.values()) + " |", "|---|" + "---:|" * len(names)]
    for rn in ("items", "last", "kv", "owners", "ffn"):
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
    # The traced step is the launch's last: its context is context + steps.
    ctx = args.context + args.steps
    roles = block_roles(shape, t.shape[0], ctx, ctx)
    print(f"# Persistent decode phase timeline: Qwen2-0.5B shape, BF16 KV, context {args.context}, step "
          f"{args.steps} of {args.steps}, {t.shape[0]} blocks, {roles['ip']} positions per item\n")
    print(report(t, roles, shape.num_layers))


if __name__ == "__main__":
    main()
