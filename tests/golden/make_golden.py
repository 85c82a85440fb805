"""Writes tests/golden/reference_pins.json: the known answers the reference's own tests hold
for this path, transcribed by hand from those tests (the C# cannot run here).

Every entry names the reference test it comes from. Run from the repository root:
    python tests/golden/make_golden.py
The output is data (inputs and expected outputs); nothing here executes reference code.
"""
import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def iq2xxs_hand_block():
    # tests/IQuantTests.cs:330-351: d = 1 (0x3C00); sub-block 0 uses grid words 0..3, sign
    # indices 0, 1, 2, 127 and scale nibble 3 (db = 0.875); every other byte is zero.
    blk = [0] * 66
    blk[0], blk[1] = 0x00, 0x3C
    blk[2], blk[3], blk[4], blk[5] = 0, 1, 2, 3
    aux1 = (3 << 28) | (0 << 0) | (1 << 7) | (2 << 14) | (127 << 21)
    for i in range(4):
        blk[6 + i] = (aux1 >> (8 * i)) & 0xFF
    want = [0.0] * 256
    for j in range(8):
        want[j] = 0.875 * 8                                              # group 0: +7.0
        want[8 + j] = 0.875 * (43 if j == 0 else 8) * (-1 if j in (0, 7) else 1)
        want[16 + j] = 0.875 * (25 if j < 2 else 8) * (-1 if j in (1, 7) else 1)
        want[24 + j] = -0.875 * (43 if j == 1 else 8)
    for e in range(32, 256):
        want[e] = 1.0                                                    # db = 0.125, grid byte 8
    return {"source": "tests/IQuantTests.cs:330-351", "block": blk, "want": want}


def route_cases():
    # tests/MoeTests.cs:116-149 (RoutingMath).
    z = math.exp(1) + math.exp(3) + math.exp(2) + 1
    p1, p2 = math.exp(3) / z, math.exp(2) / z
    return {
        "source": "tests/MoeTests.cs:116-149",
        "tol": 1e-6,
        "cases": [
            {"logits": [1, 3, 2, 0], "k": 2, "renorm": False, "sel": [1, 2], "wts": [p1, p2],
             "count": [0, 1, 1, 0]},
            {"logits": [1, 3, 2, 0], "k": 2, "renorm": True, "sel": [1, 2],
             "wts": [p1 / (p1 + p2), p2 / (p1 + p2)], "count": [0, 1, 1, 0]},
            {"logits": [2, 2, 2, 2], "k": 2, "renorm": False, "sel": [0, 1], "wts": [0.25, 0.25],
             "count": [1, 1, 0, 0]},
            {"logits": [2, 2, 2, 2], "k": 2, "renorm": True, "sel": [0, 1], "wts": [0.5, 0.5],
             "count": [1, 1, 0, 0]},
            {"logits": [1, 3, 2, 0], "k": 4, "renorm": True, "sel": [1, 2, 0, 3], "wts_sum": 1.0,
             "count": [1, 1, 1, 1]},
            {"logits": [0, 5, 0, 0], "k": 1, "renorm": True, "sel": [1], "wts": [1.0], "exact": True,
             "count": [0, 1, 0, 0]},
            {"logits": [9, 0, 0, 0], "k": 1, "renorm": True, "sel": [0], "wts": [1.0], "exact": True,
             "count": [1, 0, 0, 0]},
        ],
    }


def tables():
    # tests/IQuantTests.cs:251-317 (Tables) and src/Gguf.cs:19-66 (ids and layouts).
    return {
        "source": "tests/IQuantTests.cs:51,251-317",
        "kmask": [1 << i for i in range(8)],
        "kvalues": [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
        "iq2xxs_grid_fnv1a64": "0xbb4ee025b5ac6e8e",
        "iq2xxs_grid_spots": {"0": "0x0808080808080808", "1": "0x080808080808082b",
                              "3": "0x0808080808082b08"},
        "iq2xxs_grid_bytes": [8, 0x19, 0x2B],
        # tests/IQuantTests.cs:263,276,278 (the iq2s and iq3s grids' hashes and iq3s's ends)
        "iq2s_grid_fnv1a64": "0x123edd38a3b62b90",
        "iq3s_grid_fnv1a64": "0xfa37020c25b44829",
        "iq3s_grid_spots": {"0": "0x01010101", "1": "0x01010103", "511": "0x0f0f0101"},
        "ids": {"f32": 0, "f16": 1, "q4_0": 2, "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "q2_K": 10,
                "q3_K": 11, "q4_K": 12, "q5_K": 13, "q6_K": 14, "iq2_xxs": 16, "iq4_nl": 20, "iq3_s": 21,
                "iq2_s": 22, "iq4_xs": 23, "bf16": 30},
        "layouts": {"q4_0": [32, 18], "q4_1": [32, 20], "q5_0": [32, 22], "q5_1": [32, 24],
                    "q8_0": [32, 34], "q2_K": [256, 84], "q3_K": [256, 110], "q4_K": [256, 144],
                    "q5_K": [256, 176], "q6_K": [256, 210], "iq2_xxs": [256, 66], "iq4_nl": [32, 18],
                    "iq4_xs": [256, 136], "f32": [1, 4], "f16": [1, 2], "bf16": [1, 2], "iq3_s": [256, 110],
                    "iq2_s": [256, 82]},
        "layout_source": "src/Gguf.cs:30-66; tests/IQuantTests.cs:75-82,375-380",
    }


def quantizer_pins():
    # tests/FastMathTests.cs:44-69 (ActivationQuantizers): x = (i-16)*0.5, amax 8.
    return {
        "source": "tests/FastMathTests.cs:44-69",
        "q8_0_x": [(i - 16) * 0.5 for i in range(32)],
        "q8_0_q0": -127, "q8_0_q16": 0,
        "q8_k_x": [6.0 if i == 10 else float((i % 7) - 3) for i in range(256)],
        "q8_k_q10": -127, "q8_k_dq10": 6.0, "q8_k_tol": 1e-5,
    }


# Tiny models whose weights use this path's formats (TinyModels.StandardSpecs, tests/TinyModels.cs:166-177).
TINY_KEYS = ["llama-q4_K", "llama-q6_K", "llama-q8_0", "llama-q8_0-spm", "qwen2-q8_0", "qwen3-q4_K",
             "qwen2-q6_K-tied", "llama-f32", "llama-f16", "llama-bf16", "llama-q4_0", "llama-q4_1",
             "llama-q5_0", "llama-q5_1", "llama-q2_K", "llama-q3_K", "llama-q5_K"]
LLAMA_CPP_FIXTURE = "/root/reference/tests/fixtures/llama-cpp-reference.txt"


def llama_cpp_rows():
    """The 'argmax' and 'last' rows of the reference's llama.cpp fixture for TINY_KEYS: the top
    token at each of the 12 probe positions and the last position's logits (4 decimals), which
    tests/Tests.cs:250-278 compares against."""
    rows, key = {}, None
    with open(LLAMA_CPP_FIXTURE, encoding="utf-8") as f:
        for line in f:
            parts = line.split()
            if not parts:
                continue
            if parts[0] == "model":
                key = parts[1]
            elif key in TINY_KEYS and parts[0] in ("argmax", "last"):
                vals = [int(v) for v in parts[1:]] if parts[0] == "argmax" else [float(v) for v in parts[1:]]
                rows.setdefault(key, {})[parts[0]] = vals
    return {"source": "tests/fixtures/llama-cpp-reference.txt (llama-cpp-python 0.3.36, CPU)", "models": rows}


def main():
    out = {"iq2xxs_hand": iq2xxs_hand_block(), "route": route_cases(), "tables": tables(),
           "quantizers": quantizer_pins()}
    with open(os.path.join(HERE, "reference_pins.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    if os.path.exists(LLAMA_CPP_FIXTURE):
        with open(os.path.join(HERE, "llama_cpp_tiny.json"), "w") as f:
            json.dump(llama_cpp_rows(), f)
            f.write("\n")


if __name__ == "__main__":
    main()
