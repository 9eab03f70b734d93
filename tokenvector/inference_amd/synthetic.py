"""Synthetic tensors for benchmarks: the reference's seeded Gaussian noise.

`gi_noise` is the LCG31 + Box-Muller generator of the reference's GPT-2
driver (tv/training/gpt2_ref.tkv:1977-1991, `_gi_noise`, with its fixed 0.02
replaced by `sigma`): state s <- (1103515245 s + 12345) mod 2^31, two states
per value, u1 = (s1 + 0.5) / 2^31, u2 = s2 / 2^31,
value = f32(sqrt(0 - 2 ln u1) * cos(2 pi u2) * sigma).  The recurrence is
evaluated in parallel with numpy by doubling its affine step map, so tensors
of 10^8 elements take seconds instead of a scalar loop.

`add_outliers` overwrites round(frac * n) distinct positions, drawn from a
second LCG31 stream (pos = floor(s * n / 2^31), repeats skipped), with
gi_noise(n_out, seed2, sigma) values in draw order (the configs[1] outlier
recipe).
"""
import numpy as np

_A = 1103515245
_C = 12345
_MASK = (1 << 31) - 1


def lcg31_states(seed: int, count: int) -> np.ndarray:
    """The `count` LCG31 states that follow `seed` (seed itself excluded)."""
    out = np.empty(int(count), dtype=np.uint64)
    if count <= 0:
        return out
    out[0] = (_A * (int(seed) % (1 << 31)) + _C) & _MASK
    a, c, have = _A, _C, 1  # (a, c): the map of `have` steps
    while have < count:
        m = min(have, count - have)
        out[have:have + m] = (np.uint64(a) * out[:m] + np.uint64(c)) & np.uint64(_MASK)
        a, c = (a * a) & _MASK, (a * c + c) & _MASK
        have += m
    return out


def gi_noise(n: int, seed: int, sigma: float) -> np.ndarray:
    s = lcg31_states(seed, 2 * int(n)).astype(np.float64)
    u1 = (s[0::2] + 0.5) / 2147483648.0
    u2 = s[1::2] / 2147483648.0
    del s
    r = np.sqrt(0.0 - 2.0 * np.log(u1))
    r *= np.cos(6.283185307179586 * u2)
    r *= float(sigma)
    return r.astype(np.float32)


def add_outliers(x: np.ndarray, frac: float, seed: int, seed2: int, sigma: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    n = x.size
    n_out = min(int(round(n * frac)), n)
    if n_out <= 0:
        return x
    vals = gi_noise(n_out, seed2, sigma)
    taken = set()
    pos = []
    s = int(seed) % (1 << 31)
    while len(pos) < n_out:
        for st in lcg31_states(s, 2 * (n_out - len(pos)) + 16).tolist():
            p = (st * n) >> 31
            if p not in taken:
                taken.add(p)
                pos.append(p)
                if len(pos) == n_out:
                    break
        s = st
    x[np.asarray(pos, dtype=np.int64)] = vals
    return x
