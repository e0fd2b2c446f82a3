"""CPU test of the phase-breakdown tool's analysis (4pe_u250_amd/phase_stamps.py)
on a synthetic launch whose stamps have known phases: 16 split workgroups of
8 waves, the odd-indexed ones merging, dispatched round robin with XCD =
(index + 7) mod 8."""
import importlib

import numpy as np
import pytest

ps = importlib.import_module("4pe_u250_amd.phase_stamps")


def _synthetic_launch(nwg=16, waves=8):
    ph = np.zeros((nwg, 8), np.uint64)
    wv = np.zeros((nwg, 16, 2), np.uint64)
    index = np.arange(nwg)
    for i in range(nwg):
        entry = 1000 + i
        merger = i % 2 == 1
        ph[i, 0] = entry
        ph[i, 1] = entry + 200
        ph[i, 2] = entry + 600
        ph[i, 3] = entry + 680
        ph[i, 4] = entry + 780 if merger else 0
        ph[i, 5] = entry + 820 if merger else 0
        ph[i, 6] = 2 | (1 if merger else 0)
        ph[i, 7] = (i + 7) % 8
        for w in range(waves):
            wv[i, w, 0] = entry + 250 + 10 * w
            wv[i, w, 1] = entry + 500 + 10 * w
    return ph, wv, index


def test_launch_phases_on_known_stamps():
    ph, wv, index = _synthetic_launch()
    d = ps.launch_phases(ph, wv, len(index), index=index)
    assert d["start_max"] == pytest.approx(0.15)                  # entries 0 .. 15 ticks after the first
    assert d["first_loads_p50"] == pytest.approx(2.0 + 0.075)
    assert d["lds_merge_max"] == pytest.approx(6.15)
    assert d["arrival_p50"] == pytest.approx(0.8)
    assert d["merge_p50"] == pytest.approx(1.0)
    assert d["epilogue_p50"] == pytest.approx(0.4)
    assert d["span"] == pytest.approx(8.35)                       # the last merger: entry 15 + 820 ticks
    assert d["dispatch_xcd_offset"] == 7
    assert d["mergers"] == 8 and d["mergers_on_odd_xcd"] == 0     # odd indices land on even XCDs
    assert d["xcd_workgroups"] == [2] * 8
    assert d["first_block_spread_p50"] == pytest.approx(0.7)
    assert d["wave_first_block_mean"] == pytest.approx([2.575 + 0.1 * w for w in range(8)])
    assert d["wave_scan_end_mean"] == pytest.approx([5.075 + 0.1 * w for w in range(8)])


def test_launch_phases_flags_a_mixed_dispatch_order():
    ph, wv, index = _synthetic_launch()
    ph[3, 7] = 0                                                  # one workgroup off the round robin
    d = ps.launch_phases(ph, wv, len(index), index=index)
    assert d["dispatch_xcd_offset"] == -1
