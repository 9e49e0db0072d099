"""Writes the small golden fixtures under tests/golden/.

philox4x64_numpy.json: raw Philox4x64-10 words from numpy.random.Philox (an
implementation independent of this repository) for several (key, counter)
pairs. numpy increments the counter before each block, so random_raw() word i
with counter c0 corresponds to block counter c0 + 1 + i // 4.

Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

CASES = [
    {"key": [0, 0], "counter": [0, 0, 0, 0], "n": 8},
    {"key": [0x1234, 0x5678], "counter": [1, 2, 3, 4], "n": 8},
    {"key": [7, 0x5EC], "counter": [0, 0, 0, 0], "n": 12},
    {"key": [0xFFFFFFFFFFFFFFFF, 1], "counter": [0xFFFFFFFFFFFFFFFE, 0, 0, 0], "n": 8},
]


def main():
    out = []
    for c in CASES:
        g = np.random.Philox(key=np.array(c["key"], dtype=np.uint64), counter=np.array(c["counter"], dtype=np.uint64))
        words = [int(w) for w in g.random_raw(c["n"])]
        out.append({**c, "words": [f"{w:016x}" for w in words]})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "philox4x64_numpy.json")
    with open(path, "w") as f:
        json.dump({"generator": f"numpy {np.__version__} random.Philox", "cases": out}, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
