"""Deterministic synthetic inputs: SplitMix64 -> uniform, Box-Muller -> normal.

The same host bytes are uploaded to the GPU and handed to the CPU checker,
so parity never depends on a device RNG (the reference's cuRAND XORWOW
sequences are not pinned by any of its tests).
"""
import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed, start, count):
    """Outputs start .. start+count-1 of the SplitMix64 stream for `seed`."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(shape, low, high, seed, dtype=np.float32):
    """U[low, high) with 24 random mantissa bits, computed in float64."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype)
    for s in range(0, n, _CHUNK):
        c = min(_CHUNK, n - s)
        u = (splitmix64(seed, s, c) >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
        out[s:s + c] = (low + (high - low) * u).astype(dtype)
    return out.reshape(shape)


def normal(shape, mean, std, seed, dtype=np.float32):
    """N(mean, std^2) by Box-Muller over pairs of 53-bit uniforms."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype)
    pairs = (n + 1) // 2
    for s in range(0, pairs, _CHUNK):
        c = min(_CHUNK, pairs - s)
        bits = splitmix64(seed, 2 * s, 2 * c)
        u = (bits >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        u1, u2 = u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log1p(-u1))
        t = 2.0 * np.pi * u2
        z = np.empty(2 * c)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        lo = 2 * s
        hi = min(n, lo + 2 * c)
        out[lo:hi] = (mean + std * z[:hi - lo]).astype(dtype)
    return out.reshape(shape)


def integers(shape, low, high, seed, dtype=np.int32):
    """Uniform integers in [low, high)."""
    n = int(np.prod(shape))
    span = np.uint64(high - low)
    vals = (splitmix64(seed, 0, n) % span).astype(np.int64) + low
    return vals.astype(dtype).reshape(shape)
