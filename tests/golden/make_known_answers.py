"""Writes reference_known_answers.json: the known answers that the reference's own tests hold for
this path, as data (inputs and expected outputs), each with the test it comes from.

    python tests/golden/make_known_answers.py

Nothing here imports or runs the reference: the values are the literals of its tests, and the
two generated vectors follow the rule stated in those tests (paths relative to the reference root).
"""
import json
import math
from pathlib import Path


def e4m3_levels():
    # tests/test_trellis.py:49-51: the 127 finite E4M3 magnitudes, code c = 8 e + f
    out = []
    for c in range(127):
        e, f = c >> 3, c & 7
        out.append(f * 2.0 ** -9 if e == 0 else (8 + f) * 2.0 ** (e - 10))
    return out


def main():
    lv = e4m3_levels()
    mids = [(lv[i] + lv[i + 1]) / 2 for i in range(126)]
    # tests/test_trellis.py:52: each midpoint rounds to the level with the even code
    tie_even = [lv[i + (i & 1)] for i in range(126)]
    data = {
        "codebook": {
            "source": "tests/test_trellis.py:63",
            "state": 0,
            "value": 1.875,
        },
        "e4m3_midpoints": {
            "source": "tests/test_trellis.py:48-54 (midpoints tie to the even code, sign symmetric)",
            "inputs": mids,
            "expected": tie_even,
        },
        "e4m3_saturation": {
            "source": "tests/test_trellis.py:56-57",
            "inputs": [500.0, -500.0, "inf", "-inf"],
            "expected": [448.0, -448.0, 448.0, -448.0],
            "negative_zero_keeps_sign": True,
        },
        "resident_bytes": {
            "source": "tests/test_experts.py:116 (one 128x128 K4 projection: packed bytes + in/out fp16 side vectors)",
            "in_features": 128, "out_features": 128, "k": 4, "experts": 257,
            "per_projection_bytes": 8192 + 2 * 128 * 2,
        },
        "fp32_accumulation": {
            "source": "tests/test_fast_prefill.py:208-228 (all-zero K4 bitstream: every weight is codebook[0]; "
                      "x holds 10*sqrt(128) at every 128th position; unit scales)",
            "width": 6144, "output": 128, "spike": 10 * math.sqrt(128),
            "inner_sum": 6144 * 10 * 1.875,
            "expected_col0": 6144 * 10 * 1.875 * math.sqrt(128),
            "expected_other_cols": 0.0,
            "fp16_max": 65504.0,
        },
    }
    out = Path(__file__).with_name("reference_known_answers.json")
    out.write_text(json.dumps(data, indent=1) + "\n")
    print(out)


if __name__ == "__main__":
    main()
