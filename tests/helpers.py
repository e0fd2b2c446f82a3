"""Shared deterministic input generators for the tests and the golden script.

All generators are explicit integer arithmetic (splitmix64) so their output
does not depend on the numpy version.
"""
import numpy as np

_M64 = (1 << 64) - 1


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n consecutive splitmix64 outputs for a seed (uint64 array)."""
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & _M64) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def q17_uniform(seed: int, shape, span_bits: int = 18) -> np.ndarray:
    """Q15.17 integers uniform in [-2^span_bits, 2^span_bits)."""
    n = int(np.prod(shape))
    z = splitmix64(seed, n)
    v = (z >> np.uint64(64 - span_bits - 1)).astype(np.int64) - (1 << span_bits)
    return v.astype(np.int32).reshape(shape)


def f32_normal(seed: int, shape) -> np.ndarray:
    """FP32 ~N(0,1) by Box-Muller on splitmix64 uniforms (float64 math)."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    z = splitmix64(seed, 2 * m)
    u1 = ((z[:m] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (z[m:] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return out.astype(np.float32).reshape(shape)


def kat_vector(seed: int) -> np.ndarray:
    """The reference KAT generator (_rtl_check/linear_4pe_reduction_cosim/
    tb_attention_pe0_kv_rtl.cpp:21-31) for the 1024 channels of one PE."""
    i = np.arange(1024, dtype=np.uint64)
    raw = (i * np.uint64(37 + seed) + np.uint64(seed * 101)) % np.uint64(458753)
    return (raw.astype(np.int64) - 229376).astype(np.int32)
