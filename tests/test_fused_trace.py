"""The persistent-decode phase report (cheetah_amd/fused_trace.py) on a
synthetic stamp table: block roles as the launcher assigns them, and each
critical-path segment recovered from stamps placed at known times."""
import numpy as np

from cheetah_amd import configs, fused_trace


def test_block_roles_partition_the_grid():
    roles = fused_trace.block_roles(configs.QWEN2_0_5B, 256, 544, 640)
    # 152 FFN blocks of exactly 32 gate/up rows (4864 = 152 x 32; at most
    # 5/8 of the grid), 112 of them owners of 8 residual rows; 128 K/V
    # rotation pairs over 16 KV blocks; the items below them: 14 q heads x 5
    # runs of 128 positions
    # (640 positions fit 5 runs of 128 in the 80 item blocks). Run s of head
    # h sits at block 16 s + slot(h): every run of a head on one XCD, and
    # the 7 heads of each KV group on their own 4 XCDs (2 heads per XCD).
    assert roles["ip"] == 128
    slot = fused_trace.item_slots(14, 2)
    assert sorted(slot) == sorted(set(slot)) and all(0 <= j < 16 for j in slot)
    assert [{slot[h] % 8 for h in range(g * 7, g * 7 + 7)} for g in range(2)] == [{0, 1, 2, 3}, {4, 5, 6, 7}]
    assert roles["items"] == [16 * s + slot[h] for s in range(5) for h in range(14)]
    assert roles["last"] == [64 + slot[h] for h in range(14)]
    assert roles["kv"] == list(range(88, 104))
    assert roles["owners"] == list(range(104, 216))
    assert roles["ffn"] == list(range(104, 256))
    # Shorter launches take shorter runs: 320 positions in 5 runs of 64
    # (the 80 item blocks hold 5 runs of each of the 14 q heads).
    short = fused_trace.block_roles(configs.QWEN2_0_5B, 256, 200, 320)
    assert short["ip"] == 64 and short["items"] == [16 * s + slot[h] for s in range(4) for h in range(14)]
    # Without a fitting KV-group split, head h keeps slot h.
    assert fused_trace.item_slots(12, 3) == list(range(12))


def test_report_recovers_known_segments():
    shape = configs.QWEN2_0_5B
    L, nb = shape.num_layers, 256
    roles = fused_trace.block_roles(shape, nb, 544, 640)
    # Stamps in 100 MHz ticks: layer l starts at 2,000 l ticks (20 us per
    # layer); within a layer slot k fires at 100 k ticks (1 us apart), the
    # same in every block.
    t = np.zeros((nb, 16 * L + 3))
    for l in range(L):
        for k in range(16):
            t[:, 16 * l + k] = 1 + 2000 * l + 100 * k
    t[:, 16 * L:] = 1 + 2000 * L + np.array([0, 100, 200])
    out = fused_trace.report(t, roles, L)
    assert "mean span 20.00 us per layer" in out
    rows = {}
    for line in out.splitlines():
        cells = [c.strip() for c in line.split("|")]
        if len(cells) == 6 and cells[1] and cells[2] not in ("", "mean us", "---:"):
            rows[cells[1]] = float(cells[2])
    # q dot: slot 2 - slot 1; items -> owners: C.in (8) - P1.out (6).
    assert rows["q dot"] == 1.0
    assert rows["hand-off items -> owners"] == 2.0
    assert rows["merge + residual"] == 1.0
    # owners -> next layer's items: the next layer's P1.in (20 us + slot 1)
    # - E.out (slot 14).
    assert rows["hand-off owners -> items (+ norm)"] == 7.0
    # The segments tile the layer: their sum is the span.
    assert rows["sum"] == 20.0
