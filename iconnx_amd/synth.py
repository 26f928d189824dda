"""Seeded synthetic inputs for the BASELINE configurations (host numpy arrays).

The Gaussian generator restates the reference's test helper ``seeded(n, seed)``
(tests/common/ort_parity.rs:141-169): a SplitMix64 stream (state += 0x9E3779B97F4A7C15,
then the xor-shift-multiply finaliser), 53-bit open-interval uniforms
``(bits + 1) / (2^53 + 1)``, and Box-Muller pairs (r cos t, r sin t) cast to f32.  The
SplitMix64 state after i steps is seed + i * golden, so the stream is computed vectorised.
Uniform integers draw from the same stream: ``lo + z % (hi - lo + 1)``.
"""
import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(n, seed):
    """The first n outputs of SplitMix64 seeded with ``seed`` (uint64 array)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def seeded_normal(n, seed, mean=0.0, std=1.0):
    """n samples of N(mean, std) as float32 (the reference's ``seeded`` for mean 0, std 1)."""
    pairs = (n + 1) // 2
    z = splitmix64(2 * pairs, seed)
    u = ((z >> np.uint64(11)).astype(np.float64) + 1.0) / (float(1 << 53) + 1.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    out = out[:n].astype(np.float32)
    if mean != 0.0 or std != 1.0:
        out = (out.astype(np.float64) * std + mean).astype(np.float32)
    return out


def seeded_uniform_int(n, seed, lo, hi):
    """n integers uniform in [lo, hi] (int64)."""
    z = splitmix64(n, seed)
    return (z % np.uint64(hi - lo + 1)).astype(np.int64) + lo


def seeded_uniform_u8(n, seed):
    """n bytes uniform in [0, 255]: the little-endian bytes of the SplitMix64 stream."""
    return splitmix64((n + 7) // 8, seed).view(np.uint8)[:n].copy()


def seeded_uniform(n, seed, lo, hi):
    """n floats uniform in [lo, hi) as float32."""
    z = splitmix64(n, seed)
    u = (z >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    return (lo + (hi - lo) * u).astype(np.float32)
