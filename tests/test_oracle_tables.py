"""Pins the oracle's I-quant tables and type layouts against the reference test's own checks
(tests/IQuantTests.cs:251-317, 373-422), held in tests/golden/reference_pins.json."""
import json
import os

import numpy as np

import oracle

PINS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))


def fnv1a64(words):
    h = 14695981039346656037
    for v in words:
        for j in range(8):
            h ^= (int(v) >> (8 * j)) & 0xFF
            h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def test_iq2xxs_grid_hash_spots_and_bytes():
    t = PINS["tables"]
    grid = oracle.iq2xxs_grid()
    assert grid.size == 256
    assert fnv1a64(grid) == int(t["iq2xxs_grid_fnv1a64"], 16)
    for i, v in t["iq2xxs_grid_spots"].items():
        assert int(grid[int(i)]) == int(v, 16)
    allowed = set(t["iq2xxs_grid_bytes"])
    for g in grid:
        assert {(int(g) >> (8 * j)) & 0xFF for j in range(8)} <= allowed
    assert len(set(int(g) for g in grid)) == 256


def test_ksigns_parity_and_kvalues():
    ks = oracle.ksigns()
    for i in range(128):
        bits = bin(i).count("1")
        assert ks[i] == i | ((bits & 1) << 7)
        assert bin(int(ks[i])).count("1") % 2 == 0
    assert list(oracle.kvalues()) == PINS["tables"]["kvalues"]


def test_layouts():
    t = PINS["tables"]
    for name, (be, bb) in t["layouts"].items():
        tid = t["ids"][name]
        assert oracle.LAYOUT[tid] == (be, bb)
        assert oracle.lib().wlo_can_decode(tid) == 1
    # types outside this path are refused (src/Quants.cs:51)
    for tid in (9, 15, 17, 18, 19, 21, 22, 29):
        assert oracle.lib().wlo_can_decode(tid) == 0
        x = np.zeros(256, np.float32)
        try:
            oracle.decode(tid, np.zeros(1024, np.uint8), 256)
            assert False, "decode of an unsupported type must fail"
        except NotImplementedError:
            pass
