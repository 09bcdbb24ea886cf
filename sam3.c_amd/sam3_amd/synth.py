"""Seeded synthetic inputs shared by the GPU runs and the CPU oracle.

The reference has no N(mu, sigma) generator (its benches use xorshift32
uniforms, src/bench/bench_kernels.c:84-116), so this module defines one:
SplitMix64 (counter form) -> 53-bit uniforms -> Box-Muller in float64 ->
float32. Both the HIP path and the oracle are fed the very same arrays.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n, offset=0):
    """Outputs offset+1 .. offset+n of SplitMix64 started at ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed, n):
    """n doubles in [0, 1)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def randn(seed, shape, std=1.0, mean=0.0, chunk=1 << 22):
    """float32 N(mean, std^2) of the given shape, deterministic in ``seed``."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    npairs = (n + 1) // 2
    for p0 in range(0, npairs, chunk):
        p1 = min(npairs, p0 + chunk)
        bits = splitmix64(seed, 2 * (p1 - p0), offset=2 * p0)
        u = (bits >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        u1, u2 = 1.0 - u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        th = 2.0 * np.pi * u2
        z = np.empty(2 * (p1 - p0))
        z[0::2] = r * np.cos(th)
        z[1::2] = r * np.sin(th)
        lo, hi = 2 * p0, min(n, 2 * p1)
        out[lo:hi] = (z[: hi - lo] * std + mean).astype(np.float32)
    return out.reshape(shape)


def tensor_seed(config_seed, tensor_id):
    """One independent stream per tensor: seed = config seed + tensor id."""
    return (config_seed * 1000003 + tensor_id) & 0xFFFFFFFFFFFFFFFF
