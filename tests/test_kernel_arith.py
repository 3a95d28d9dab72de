"""Integer arithmetic the decode kernels do in floating point (CPU).

`floor_div` in aiproj_amd/csrc/kvfp8_decode_mfma.hip computes floor(n / d) for
0 <= n < 2^53, d >= 1 as the truncation of one IEEE double division. Python floats
are IEEE doubles with correctly rounded division, so the same expression here checks
the claim: exact against integer division at the operand ranges the kernels use
(w * total and (x + 1) * groups - 1 below 2^42, tiles below 2^31), at exact multiples
and one below them, and up to the 2^53 bound.
"""

from __future__ import annotations

import random


def floor_div(n: int, d: int) -> int:
    return int(float(n) / float(d))


def test_floor_div_exact_at_multiples_and_neighbours():
    rng = random.Random(11)
    for _ in range(20000):
        d = rng.randrange(1, 1 << 31)
        k = rng.randrange(0, (1 << 42) // d + 1)
        for n in (k * d - 1, k * d, k * d + 1, k * d + d - 1):
            if 0 <= n < (1 << 53):
                assert floor_div(n, d) == n // d, (n, d)


def test_floor_div_exact_on_random_operands_up_to_two_to_the_53():
    rng = random.Random(12)
    for bits in (20, 31, 42, 52, 53):
        for _ in range(20000):
            n = rng.randrange(0, 1 << bits)
            d = rng.randrange(1, 1 << rng.choice((1, 11, 31, 40)))
            assert floor_div(n, d) == n // d, (n, d)


def test_group_split_round_trip():
    # The decode kernel's equal-tile split and the combine's inverse: workgroup w
    # takes [floor(w T / G), floor((w + 1) T / G)); group_of(x) = floor(((x + 1) G - 1) / T)
    # is the workgroup whose range holds tile x.
    rng = random.Random(13)
    for _ in range(300):
        total = rng.randrange(1, 1 << 31)
        groups = rng.randrange(1, 2049)
        for w in rng.sample(range(groups), min(groups, 8)):
            start = floor_div(w * total, groups)
            end = floor_div((w + 1) * total, groups)
            assert start == w * total // groups and end == (w + 1) * total // groups
            for x in {start, end - 1}:
                if start <= x < end:
                    assert floor_div((x + 1) * groups - 1, total) == w
