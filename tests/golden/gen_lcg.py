"""Writes tests/golden/lcg.json: the first values of the reference's KAT generator
(Tests/DictatorEngineTests/GemmTests.swift:7-14) for the seeds the reference tests use, computed
with Python integers (no oracle involved)."""
import json
import os

SEEDS = [1, 2, 11, 12, 13, 21, 22, 41, 42, 46, 51, 61]


def lcg(n, seed):
    M = (1 << 64) - 1
    a, c = 6364136223846793005, 1442695040888963407
    s = (seed * a + c) & M
    out = []
    for _ in range(n):
        s = (s * a + c) & M
        out.append(float((s >> 11) % (1 << 24)) / float(1 << 23) - 1.0)
    return out


if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lcg.json")
    with open(path, "w") as f:
        json.dump({"generator": "GemmTests.swift:7-14", "values": {str(s): lcg(16, s) for s in SEEDS}}, f, indent=0)
    print("wrote", path)
