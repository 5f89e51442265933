"""Counter-based seeded random numbers shared by every synthetic input.

The generator is written down exactly so the same streams can be reproduced in
any language: output i (i = 1, 2, ...) of stream `seed` is splitmix64 applied to
the state `seed + i * 0x9E3779B97F4A7C15` (mod 2**64).  Uniform doubles take
the top 53 bits; normals use Box-Muller with two consecutive uniforms
(u1 = 1 - u[2j], u2 = u[2j+1], z = sqrt(-2 ln u1) cos(2 pi u2)).
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z):
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed, n):
    """First `n` outputs of splitmix64 started at state `seed` (uint64 array)."""
    i = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN)


def derive_seed(base, *keys):
    """Sub-stream seed: fold each integer key into the base with splitmix64."""
    s = int(base) & 0xFFFFFFFFFFFFFFFF
    for k in keys:
        s = int(splitmix64(s ^ (int(k) & 0xFFFFFFFFFFFFFFFF), 1)[0])
    return s


def uniform(seed, n):
    """n doubles in [0, 1)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed, n):
    """n standard normal doubles (Box-Muller, cosine branch)."""
    u = uniform(seed, 2 * n)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
