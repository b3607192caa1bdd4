"""Host logic of the isolated-layer bench (hffn_amd.bench_ffn): the dense control's weights, the float64 gate, the
A/A verdict and the ratios."""
from __future__ import annotations

import numpy as np

from hffn_amd import bench_ffn, synth
from oracle import reference


def test_dense_weights_and_gate_match_the_oracle():
    layer = synth.make_layer(synth.CASES["irreg_512_2048"])
    w_up, w_down = bench_ffn.dense_weights(layer)
    ref_up, ref_down = reference.dense_weights(layer)
    assert np.array_equal(w_up, ref_up.astype(np.float32)) and np.array_equal(w_down, ref_down.astype(np.float32))
    x = synth.make_input(synth.CASES["irreg_512_2048"], 5)
    assert np.abs(bench_ffn.float64_forward(layer, x, w_up, w_down) - reference.forward(layer, x)).max() < 1e-12


def _cell(layer, n, hffn, hffn_copy, dense, dense_copy, gates=True):
    """A worker's cell record: the schedule's observations, the windows of each arm taking its given values in turn."""
    values = {"hffn": list(hffn), "hffn_copy": list(hffn_copy), "dense": list(dense), "dense_copy": list(dense_copy)}
    observations = [{"block": b, "slot": s, "arm": arm, "us": values[arm].pop()} for b, s, arm in bench_ffn.schedule()]
    return {"layer": layer, "n": n, "observations": observations, "modes": ["tiles", "tiles"],
            "gates": {"oracle": gates, "copy_bitwise": True, "memory_steady": True}}


def test_summary_reads_ratios_only_when_admissible():
    cells = [_cell("a", 1, [10.0] * 4, [10.2] * 4, [20.0] * 4, [19.8] * 4), _cell("a", 1, [11.0] * 4, [11.0] * 4, [21.0] * 4, [21.5] * 4)]
    s = bench_ffn.summarise(cells)
    assert s["admissible"] and s["aa"]["hffn"] == {"within": 2, "of": 2, "max_abs_dev": 0.0196}
    row = s["cells"][0]
    assert row["sessions"] == 2 and row["hffn_over_dense"]["min"] == 0.5 and abs(row["hffn_over_dense"]["max"] - 11 / 21) < 1e-4
    bad = bench_ffn.summarise(cells + [_cell("a", 4, [10.0] * 4, [10.5] * 4, [20.0] * 4, [20.0] * 4)])
    assert not bad["admissible"] and "hffn_over_dense" not in bad["cells"][0]
    failed = bench_ffn.summarise([_cell("a", 1, [10.0] * 4, [10.0] * 4, [20.0] * 4, [20.0] * 4, gates=False)])
    assert not failed["admissible"] and not failed["gates"]


def test_block_orders_balance_every_arm():
    """Each order holds every arm twice with the same mean position (equal time centroid), and the two orders
    together put each arm first once in four."""
    for order in bench_ffn.BLOCK_ORDERS:
        positions = {arm: [i for i, a in enumerate(order) if a == arm] for arm in set(order)}
        assert all(len(p) == 2 and sum(p) == 7 for p in positions.values())
    assert bench_ffn.parse_cells("pythia410m_d50:2048,homog_512_2048:4") == [("pythia410m_d50", 2048), ("homog_512_2048", 4)]


def test_schedule_and_medians():
    """The schedule runs the two orders' 16 windows, every arm four times; a cell's arm medians come from its
    observations (the middle two of four windows averaged)."""
    plan = bench_ffn.schedule()
    assert len(plan) == 16 and all(sum(arm == a for _, _, arm in plan) == 4 for a in bench_ffn.ARMS)
    assert [b for b, _, _ in plan] == [0] * 8 + [1] * 8
    cell = _cell("a", 1, [1.0, 2.0, 3.0, 10.0], [1.0] * 4, [5.0] * 4, [5.0] * 4)
    assert bench_ffn.arm_medians(cell) == {"hffn": 2.5, "hffn_copy": 1.0, "dense": 5.0, "dense_copy": 5.0}
