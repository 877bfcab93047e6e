"""Sequential restatement of the reference's generator, the checker for the vectorised one.

`generator(seed)` (`webgpu/testing/deterministic-input.js:1-10`): state += 0x6d2b79f5, then
two Math.imul mixing rounds and a final xor-shift, divided by 2^32.  This walks it one draw
at a time in Python integers, exactly as the JS closure does.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
import numpy as np


def uniform_sequential(seed: int, count: int) -> np.ndarray:
    state = seed & 0xFFFFFFFF
    out = np.empty(count)
    m = 0xFFFFFFFF
    for i in range(count):
        state = (state + 0x6D2B79F5) & m
        v = state
        v = ((v ^ (v >> 15)) * (v | 1)) & m
        v = (v ^ ((v + (((v ^ (v >> 7)) * (v | 61)) & m)) & m)) & m
        out[i] = ((v ^ (v >> 14)) & m) / 4294967296.0
    return out
