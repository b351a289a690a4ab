"""The persistent-decode phase report (cheetah_amd/fused_trace.py) on a
synthetic stamp table: block roles as the launcher assigns them, and each
critical-path segment recovered from stamps placed at known times."""
import numpy as np

from cheetah_amd import configs, fused_trace


def test_block_roles_partition_the_grid():
    roles = fused_trace.block_roles(configs.QWEN2_0_5B, 256, 544)
    # 896 rows of o_proj/down over 7 rows per block; 1,152 QKV rows in pairs
    # over 7 pairs per block; 2 KV heads x 5 splits x 7 q heads items.
    assert roles["H"] == list(range(128))
    assert len(roles["Aall"]) == 83 and len(roles["Ball"]) == 70
    assert set(roles["A"]) | set(roles["AB"]) == set(roles["Aall"])
    assert set(roles["B"]) | set(roles["AB"]) == set(roles["Ball"])
    assert not set(roles["A"]) & set(roles["B"])
    assert max(roles["Ball"]) == 255


def test_report_recovers_known_segments():
    shape = configs.QWEN2_0_5B
    L, nb = shape.num_layers, 256
    roles = fused_trace.block_roles(shape, nb, 544)
    # Stamps in 100 MHz ticks: layer l starts at 2,000 l ticks (20 us per
    # layer); within a layer each slot k fires at 100 k ticks (1 us apart),
    # the same in every block.
    t = np.zeros((nb, 16 * L + 3))
    for l in range(L):
        for k in range(16):
            t[:, 16 * l + k] = 1 + 2000 * l + 100 * k
    t[:, 16 * L:] = 1 + 2000 * L + np.array([0, 100, 200])
    out = fused_trace.report(t, roles, L)
    assert "mean span 20.00 us per layer" in out
    # A dot + store: A.out (slot 2) - A.in (slot 1) = 1 us; the hand-off
    # A -> B: B.in (3) - A.out (2) = 1 us; B -> C: C.in (8) - PV (6) = 2 us.
    rows = {}
    for line in out.splitlines():
        cells = [c.strip() for c in line.split("|")]
        if len(cells) == 6 and cells[1] and cells[2] not in ("", "mean us", "---:"):
            rows[cells[1]] = float(cells[2])
    assert rows["A dot + store"] == 1.0
    assert rows["hand-off A->B"] == 1.0
    assert rows["hand-off B->C (+ merge)"] == 2.0
    # E -> next A: the next layer's A.in (20 us + slot 1) - E.out (slot 13).
    assert rows["hand-off E->A(next)"] == 8.0
    # The segments tile the layer: their sum is the span.
    assert rows["sum"] == 20.0
