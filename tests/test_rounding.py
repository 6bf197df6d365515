"""The fused GEMV's quantizer rounds with trunc(v + copysign(0.5 - 2^-25, v)) in
place of roundf.  This checks, over every non-negative float32 below 2^23, that
the two give the same integer (ties away from zero); the sign makes it symmetric.
Pure NumPy, ~20 s."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import numpy as np


def test_round_half_away_trick_exhaustive():
    c = np.float32(0.5) - np.float32(2.0 ** -25)
    assert c == np.float32(0.49999997)
    end = 0x4B000000  # 2^23
    step = 1 << 25
    bad = 0
    for start in range(0, end, step):
        v = np.arange(start, min(start + step, end), dtype=np.uint32).view(np.float32)
        fast = np.trunc(v + c)
        t = np.trunc(v)
        ref = np.where(v - t >= np.float32(0.5), t + 1, t)  # roundf for v >= 0
        bad += int(np.count_nonzero(fast != ref))
    assert bad == 0
    # negative side spot check, including ties
    v = -np.array([0.5, 1.5, 2.5, 0.49999997, 126.5, 127.0, 3.4999998], np.float32)
    fast = np.trunc(v - c)
    assert list(fast) == [-1.0, -2.0, -3.0, -0.0, -127.0, -127.0, -3.0]
