"""Q8 inputs planted at the rounding boundaries of quantize_q8_global
(kernels/gemv.cu:43-65: d = amax * fl(1/127), q = rint_even(x / d)).

Each 32-value group holds its amax at value 0; the other values sit 0-3 f32
ulps from (k + 1/2) d for random k, either sign, so x / d lands within about
2^-20 of a .5 tie, inside the window where a reciprocal-multiply quotient
can round differently from the IEEE one.  Some groups are all zero, some
have a subnormal d (amax below 127 * 2^-126), some an exact tie (x = (k +
1/2) d when that product is exact in f32)."""
import numpy as np


def near_tie_groups(n_groups: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    inv127 = np.float32(1.0) / np.float32(127.0)
    out = np.zeros((n_groups, 32), np.float32)
    for g in range(n_groups):
        kind = g % 8
        if kind == 0:
            continue  # all zero: q = 0, d = 0
        if kind == 1:
            amax = np.float32(rng.uniform(1e-40, 1.4e-36))  # d subnormal
        else:
            amax = np.float32(10.0 ** rng.uniform(-6, 4))
        d = np.float32(amax * inv127)
        row = out[g]
        row[0] = amax if rng.random() < 0.5 else -amax
        for i in range(1, 32):
            k = int(rng.integers(0, 127))
            x = np.float32((k + 0.5) * np.float64(d))
            for _ in range(int(rng.integers(0, 4))):
                x = np.nextafter(x, np.float32(np.inf) if rng.random() < 0.5 else np.float32(0))
            if abs(x) > amax:
                x = np.float32(amax)
            row[i] = -x if rng.random() < 0.5 else x
    return out.reshape(-1)
