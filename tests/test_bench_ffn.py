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
    samples = {"hffn": hffn, "hffn_copy": hffn_copy, "dense": dense, "dense_copy": dense_copy}
    return {"layer": layer, "n": n, "samples_us": samples, "modes": ["tiles", "tiles"],
            "gates": {"oracle": gates, "copy_bitwise": True, "memory_steady": True}}


def test_summary_reads_ratios_only_when_admissible():
    cells = [_cell("a", 1, [10.0] * 8, [10.2] * 8, [20.0] * 8, [19.8] * 8), _cell("a", 1, [11.0] * 8, [11.0] * 8, [21.0] * 8, [21.5] * 8)]
    s = bench_ffn.summarise(cells)
    assert s["admissible"] and s["aa"]["hffn"] == {"within": 2, "of": 2, "max_abs_dev": 0.0196}
    row = s["cells"][0]
    assert row["sessions"] == 2 and row["hffn_over_dense"]["min"] == 0.5 and abs(row["hffn_over_dense"]["max"] - 11 / 21) < 1e-4
    bad = bench_ffn.summarise(cells + [_cell("a", 4, [10.0] * 8, [10.5] * 8, [20.0] * 8, [20.0] * 8)])
    assert not bad["admissible"] and "hffn_over_dense" not in bad["cells"][0]
    failed = bench_ffn.summarise([_cell("a", 1, [10.0] * 8, [10.0] * 8, [20.0] * 8, [20.0] * 8, gates=False)])
    assert not failed["admissible"] and not failed["gates"]


def test_block_orders_balance_every_arm():
    """Each order holds every arm twice with the same mean position (equal time centroid), and the two orders
    together put each arm first once in four."""
    for order in bench_ffn.BLOCK_ORDERS:
        positions = {arm: [i for i, a in enumerate(order) if a == arm] for arm in set(order)}
        assert all(len(p) == 2 and sum(p) == 7 for p in positions.values())
    assert bench_ffn.parse_cells("pythia410m_d50:2048,homog_512_2048:4") == [("pythia410m_d50", 2048), ("homog_512_2048", 4)]
