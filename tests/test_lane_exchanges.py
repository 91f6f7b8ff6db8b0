"""The attention backward forms D = rowsum(dO o O) with the 16-lane butterfly of the former prep
kernel (each lane adds the partner value of lane ^ 8, then ^ 4, ^ 2, ^ 1), but exchanges the
values by DPP row rotations (lane + 8, + 4, + 2, + 1 mod 16) instead of xor shuffles. The kernel
comment's argument: after the step with 8 a lane's sum depends on its position mod 8 only, so
the rotation reaches a lane holding the same value as the xor partner, and so on. This CPU test
simulates both exchanges lane by lane in float32 and checks that every lane ends with the same
bits, and that a rotation applied where the argument does not hold (first step by 4) does not.
"""

from __future__ import annotations

import numpy as np


def _xor_butterfly(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.float32).copy()
    lanes = np.arange(16)
    for off in (8, 4, 2, 1):
        v = (v + v[lanes ^ off]).astype(np.float32)
    return v


def _rotation_butterfly(v: np.ndarray, order=(8, 4, 2, 1)) -> np.ndarray:
    v = v.astype(np.float32).copy()
    lanes = np.arange(16)
    for n in order:
        v = (v + v[(lanes + n) % 16]).astype(np.float32)
    return v


def _rows(seed: int, n: int = 2000) -> np.ndarray:
    rng = np.random.default_rng(seed)
    mag = rng.uniform(-30, 30, size=(n, 16))  # wide dynamic range: additions round differently
    return (rng.standard_normal((n, 16)) * np.exp2(mag)).astype(np.float32)


def test_rotations_give_the_xor_butterflys_bits():
    for row in _rows(0):
        want = _xor_butterfly(row)
        got = _rotation_butterfly(row)
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
        assert np.all(want.view(np.uint32) == want.view(np.uint32)[0])  # every lane: one value


def test_the_argument_needs_the_order():
    # Rotating by 4 first (no periodicity yet) is a different sum tree: some rows differ.
    rows = _rows(1)
    differ = sum(not np.array_equal(_xor_butterfly(r).view(np.uint32),
                                    _rotation_butterfly(r, (4, 8, 2, 1)).view(np.uint32))
                 for r in rows)
    assert differ > 0
