"""The margin metrics of the parity tests (tests/helpers.py), on values whose
f16 distances are known by construction."""
import numpy as np

from helpers import f16_ulp_distance


def test_f16_ulp_distance_known_steps():
    one = np.float16(1.0)
    nxt = np.nextafter(one, np.float16(2.0))
    assert f16_ulp_distance(nxt, 1.0) == 1
    assert f16_ulp_distance(one, 1.0) == 0
    # across zero: -min_denormal .. +min_denormal is two steps; -0 == +0
    tiny = np.float16(2.0 ** -24)
    assert f16_ulp_distance(-tiny, tiny) == 2
    assert f16_ulp_distance(np.float16(-0.0), 0.0) == 0
    # the reference value is rounded to f16 first (nearest even)
    assert f16_ulp_distance(one, 1.0 + 2.0 ** -12) == 0          # below half an ulp
    assert f16_ulp_distance(nxt, 1.0 + 2.0 ** -10 * 0.75) == 0   # rounds up to nxt
    # at magnitude 4..8 one ulp is 2^-8
    four = np.float16(4.0)
    assert f16_ulp_distance(four + np.float16(3 * 2.0 ** -8), 4.0) == 3
    assert f16_ulp_distance(np.array([1.0, -1.0], np.float16), np.array([1.0, -1.0 - 2.0 ** -10])).tolist() == [0, 1]
