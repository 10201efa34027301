"""Writes reference_kats.json: the known-answer vectors of the reference's own unit tests.

The inputs and expected outputs are transcribed from the test bodies they cite (paths relative
to the reference repository root); blocks are rebuilt here byte for byte as those tests build
them. Run: python tests/golden/make_kats.py
"""
import json
import os
import struct

import numpy as np


def f16le(v: float) -> bytes:
    return np.array([v], np.float16).tobytes()


def main():
    kats = {}
    # crates/jevons-formats/src/quant.rs:199-208
    kats["q4k_scale_min"] = {
        "source": "crates/jevons-formats/src/quant.rs:199-208",
        "scale_bytes": [0xC1, 0x82, 0x43, 0x04, 0x85, 0xC6, 0x07, 0x48, 0x12, 0x34, 0x56, 0x78],
        "pairs": {"0": [1, 5], "4": [50, 33], "7": [8, 23]},
    }
    # crates/jevons-formats/src/quant.rs:210-218
    q8 = bytearray(34)
    q8[0:2] = f16le(0.5)
    q8[2] = (-4) & 0xFF
    q8[33] = 7
    kats["q8_0"] = {"source": "crates/jevons-formats/src/quant.rs:210-218", "block_hex": q8.hex(),
                    "expect": {"0": -2.0, "31": 3.5}}
    # crates/jevons-formats/src/quant.rs:220-225
    q5 = bytearray(22)
    q5[0:2] = f16le(1.0)
    q5[2:6] = struct.pack("<I", 1 | (1 << 16))
    q5[6] = 0x3F
    kats["q5_0"] = {"source": "crates/jevons-formats/src/quant.rs:220-225", "block_hex": q5.hex(),
                    "expect": {"0": 15.0, "16": 3.0, "1": -16.0}}
    # crates/jevons-formats/src/quant.rs:228-237
    p8 = bytearray(34)
    p8[0:2] = f16le(0.5)
    p8[2:6] = bytes([1, 2, 3, 4])
    kats["pack_q8_0"] = {"source": "crates/jevons-formats/src/quant.rs:228-237", "block_hex": p8.hex(),
                         "q_words": 8, "q0": struct.unpack("<I", bytes([1, 2, 3, 4]))[0], "d": [0.5],
                         "short_block_is_error": True}
    # crates/jevons-core/src/model.rs:221-234
    kats["greedy"] = {"source": "crates/jevons-core/src/model.rs:221-234", "cases": [
        {"logits": [1000.0, float(np.float32(1000.0) + np.log(np.float32(2.0))), 0.0],
         "index": 1, "prob": 2.0 / 3.0, "prob_tol": 1e-4},
        {"logits": [3.0, 3.0], "index": 0},
        {"logits": ["inf"], "error": True},
    ]}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(path, "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main()
