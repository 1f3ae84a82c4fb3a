"""Writes tests/golden/xorshift64.json: the reference FA test's generator
(Tests/PopcornTests/Kernels/BidirectionalFATests.swift:98-102) evaluated with
Python integers and numpy float32, independently of the C oracle."""
import json
import os

import numpy as np

MASK = (1 << 64) - 1


def xorshift(state):
    state ^= (state << 13) & MASK
    state ^= state >> 7
    state ^= (state << 17) & MASK
    return state


def main():
    seed = 0xDEADBEEFCAFEBABE
    st, outs, floats = seed, [], []
    for _ in range(16):
        st = xorshift(st)
        outs.append(f"{st:016x}")
    st = seed
    for _ in range(16):
        st = xorshift(st)
        signed = st - (1 << 64) if st >> 63 else st
        hi = signed >> 32  # arithmetic shift
        v = np.float32(hi) / np.float32(2147483647) * np.float32(0.2)
        floats.append(float(np.float32(v)))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "xorshift64.json")
    with open(path, "w") as f:
        json.dump({"seed": f"{seed:x}", "outputs": outs, "fa_test_floats": floats}, f, indent=1)


if __name__ == "__main__":
    main()
