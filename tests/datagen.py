"""Seeded synthetic inputs shaped like the benchmark configurations (numpy, host side).

Each generator returns a numpy array whose raw bytes are the tensor's bytes
(bf16 is returned as uint16 bit patterns).
"""
import numpy as np

F32, BF16, F16, I8, I32 = 0, 1, 2, 3, 4


def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 → bf16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = 0x7FC0
    return r


def normal_f32(n, sigma, seed):
    return (np.random.default_rng(seed).standard_normal(n) * sigma).astype(np.float32)


def normal_bf16(n, sigma, seed):
    return f32_to_bf16_bits(normal_f32(n, sigma, seed))


def exp_avg_sq(n, seed):
    g = normal_f32(n, 1e-3, seed)
    return (g * g + np.float32(1e-12)).astype(np.float32)


def adversarial_f32(n, seed, random_block=None):
    """Lognormal over ~30 binades with 0.1% zeros, 0.01% denormals, 0.001% ±inf/NaN and an
    optional block of uniform random bits (the incompressible case)."""
    rng = np.random.default_rng(seed)
    x = np.exp(rng.standard_normal(n) * 5.0 - 12.0).astype(np.float32)
    k = max(1, n // 1000)
    x[rng.integers(0, n, k)] = 0.0
    d = max(1, n // 10000)
    x[rng.integers(0, n, d)] = (rng.random(d) * 1e-39).astype(np.float32)
    s = max(1, n // 100000)
    idx = rng.integers(0, n, s)
    x[idx] = np.array([np.inf, -np.inf, np.nan], np.float32)[rng.integers(0, 3, s)]
    if random_block:
        a, b = random_block
        x[a:b] = rng.integers(0, 2**32, b - a, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return x


def raw_bytes(arr):
    return np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
