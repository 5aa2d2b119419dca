"""Writes tests/golden/reference_kats.json: the known-answer vectors of the reference's own CPU tests.

The values are the literal inputs and expected outputs asserted in the reference's tests/test_formats.py
(1-bit layout KAT :19-22, tail rejection :25-31, dense_weight :40-43, ternary layout KAT :52, ternary
rejections :55-59). They are data, restated here; nothing from the reference is imported or executed.
"""
import json
from pathlib import Path

KATS = {
    "pack_signs_one_hot": {  # signs = -1 everywhere except +1 at k = 3, K = 8 -> one byte 1 << 3
        "signs": [[-1, -1, -1, 1, -1, -1, -1, -1]], "codes": [[8]]},
    "tail_bits_rejected": {  # K = 12: byte 1 bit 7 is code 15, past K -> "tail"
        "codes": [[0, 128], [0, 0]], "k": 12},
    "codes_shape_rejected": {"codes_shape": [2, 2], "k": 20},  # K = 20 needs 3 bytes per row
    "dense_weight": {
        "signs": [[1, -1, 1], [-1, -1, 1]], "scale": [0.5, 2.0],
        "dense": [[0.5, -0.5, 0.5], [-2.0, -2.0, 2.0]]},
    "pack_ternary": {"values": [[0, 1, -1, 1]], "codes": [[0b01_10_01_00]]},
    "ternary_rejected": [
        {"codes": [[0b11]], "k": 4},           # the unused 11 pattern
        {"codes": [[0b01_00_00_00]], "k": 3},  # a nonzero code past K
    ],
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_kats.json")
    out.write_text(json.dumps(KATS, indent=1) + "\n")
    print(out)
