"""Writes the known-answer fixtures in this directory.

The expected values are fixed by construction (integer arithmetic and
published constants), never by running the oracle or the GPU path:

* kv_quant.json -- int8 KV quantizer cases (model/runtime.ts:697-714,
  901-907 of needle.js).  Each vector's absmax is 127 * 2**e, so the float64
  scale is exactly 2**e and every x / s is an exact half-integer j / 2; the
  expected code is the round-half-to-even of j / 2 computed on integers.  A
  zero vector pins the 1e-12 floor of the absmax.
* select.json -- selectToken / argmax cases (model/runtime.ts:880-899,
  model/math.ts:140-160) whose winners follow from the strict '>' rule by
  inspection: ties keep the earliest candidate in list order, NaN never
  replaces a best, a NaN first candidate is kept.
* splitmix64.json -- the published SplitMix64 test vector for seed 0, which
  pins the synthetic-data generator.

Run: python tests/golden/make_golden.py
"""

import json
import math
import struct
from pathlib import Path

HERE = Path(__file__).resolve().parent


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def half_even_of_half(j: int) -> int:
    """round_half_even(j / 2) on integers."""
    if j % 2 == 0:
        return j // 2
    lo, hi = (j - 1) // 2, (j + 1) // 2
    return lo if lo % 2 == 0 else hi


def kv_cases():
    cases = []
    cases.append({"name": "zero", "x": [0.0] * 64, "codes": [0] * 64,
                  "scale_bits": f32_bits(1e-12 / 127)})
    for e, sign, offset in [(-7, 1, 0), (-3, -1, 17), (0, 1, 101), (4, -1, 5), (-20, 1, 63)]:
        step = 2.0 ** e
        js = []
        for i in range(64):
            # Half-integers spread over [-254, 254] (x/s = j/2 in [-127, 127]).
            j = ((i * 37 + offset) % 509) - 254
            js.append(j)
        js[offset % 64] = 254 * sign  # absmax exactly 127 * 2**e
        js = [max(-254, min(254, j)) for j in js]
        x = [j / 2 * step for j in js]
        codes = [half_even_of_half(j) for j in js]
        cases.append({"name": f"pow2_e{e}_s{sign}", "x": x, "codes": codes,
                      "scale_bits": f32_bits(step)})
    # Every tie n + 1/2 for n in [-127, 126].
    step = 2.0 ** -5
    for start in range(-254, 254, 64):
        js = [start + i for i in range(64)]
        js = [max(-254, min(254, j)) for j in js]
        js[0] = 254  # absmax
        x = [j / 2 * step for j in js]
        cases.append({"name": f"ties_from_{start}", "x": x,
                      "codes": [half_even_of_half(j) for j in js],
                      "scale_bits": f32_bits(step)})
    return cases


def select_cases():
    nan = float("nan")
    inf = float("inf")
    return [
        {"name": "first_max_wins", "logits": [1, 3, 3, 2], "allowed": None, "id": 1},
        {"name": "list_order_tie", "logits": [5, 5, 5, 5, 1], "allowed": [3, 1, 2], "id": 3},
        {"name": "allowed_excludes_max", "logits": [9, 1, 4, 4, 2], "allowed": [1, 3, 4], "id": 3},
        {"name": "nan_first_kept", "logits": [nan, 7, 8], "allowed": None, "id": 0},
        {"name": "nan_first_in_list_kept", "logits": [1, nan, 8], "allowed": [1, 2], "id": 1},
        {"name": "nan_later_skipped", "logits": [1, nan, 0.5], "allowed": None, "id": 0},
        {"name": "neg_inf_first", "logits": [-inf, -inf, -inf], "allowed": None, "id": 0},
        {"name": "single_allowed", "logits": [3, 2, 1, 0], "allowed": [2], "id": 2},
        {"name": "signed_zero_tie", "logits": [-0.0, 0.0, -1], "allowed": None, "id": 0},
        {"name": "uniform", "logits": [0.25] * 16, "allowed": None, "id": 0,
         "log_probability": -math.log(16)},
    ]


def main():
    (HERE / "kv_quant.json").write_text(json.dumps(kv_cases(), indent=0))
    (HERE / "select.json").write_text(json.dumps(select_cases(), indent=1))
    # Published SplitMix64 outputs for seed 0 (state advanced before mixing).
    (HERE / "splitmix64.json").write_text(json.dumps({
        "seed": 0,
        "outputs": ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4", "0x06c45d188009454f",
                    "0xf88bb8a8724c81ec"],
    }, indent=1))


if __name__ == "__main__":
    main()
