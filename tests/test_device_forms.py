"""CPU checks of the closed forms the kernels evaluate in floating point where
the reference uses integer division: each must equal the integer result on the
whole range the kernel meets.  (The device evaluates them with IEEE f64; numpy
float64 with two roundings is never more accurate than the device's fma.)"""
import random

import numpy as np


def test_cdf_floor_quotient_f64():
    """floor(e*Rm/S) = floor(fma(e*Rm, 1/S, 2^-30)) for e in [1, 65535],
    0 <= Rm < S, 65535 <= S <= 2^26 (k_head_cdf step 3; the reference divides
    in u64: softmax_cdf.rs:114-120)."""
    rng = random.Random(5)
    e = np.arange(1, 65536, dtype=np.int64)
    ef = e.astype(np.float64)
    Ss = [65535, 65536, 65537, 1 << 20, (1 << 26) - 1, 1 << 26, 255255, 1000003]
    Ss += [rng.randint(65535, 1 << 26) for _ in range(60)]
    for S in Ss:
        inv = 1.0 / S
        for Rm in [0, 1, S - 1, S // 2, S // 3] + [rng.randint(0, S - 1) for _ in range(3)]:
            q = np.floor(ef * float(Rm) * inv + 2.0 ** -30).astype(np.int64)
            assert np.array_equal(q, (e * Rm) // S), (S, Rm)
