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


def _fnv1a64_bytes(words, nbytes):
    h = 0xcbf29ce484222325
    for w in words:
        for j in range(nbytes):
            h ^= (int(w) >> (8 * j)) & 0xFF
            h = (h * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_iq2s_and_iq3s_grids():
    """The reference test's hashes of Iq2sGrid and Iq3sGrid (tests/IQuantTests.cs:263,276,278)
    and Iq3sGrid's end entries; every byte in the grids' byte sets."""
    t = PINS["tables"]
    g2, g3 = oracle.iq2s_grid(), oracle.iq3s_grid()
    assert g2.size == 1024 and g3.size == 512
    assert _fnv1a64_bytes(g2, 8) == int(t["iq2s_grid_fnv1a64"], 16)
    assert _fnv1a64_bytes(g3, 4) == int(t["iq3s_grid_fnv1a64"], 16)
    for i, v in t["iq3s_grid_spots"].items():
        assert int(g3[int(i)]) == int(v, 16)
    assert all({(int(g) >> (8 * j)) & 0xFF for j in range(8)} <= {8, 0x19, 0x2B} for g in g2)
    assert all({(int(g) >> (8 * j)) & 0xFF for j in range(4)} <= set(range(1, 16, 2)) for g in g3)
    assert len(set(int(g) for g in g2)) == 1024 and len(set(int(g) for g in g3)) == 512


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
    for tid in (9, 15, 17, 18, 19, 29):
        assert oracle.lib().wlo_can_decode(tid) == 0
        x = np.zeros(256, np.float32)
        try:
            oracle.decode(tid, np.zeros(1024, np.uint8), 256)
            assert False, "decode of an unsupported type must fail"
        except NotImplementedError:
            pass
