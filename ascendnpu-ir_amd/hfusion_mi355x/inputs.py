"""Seeded, counter-based synthetic inputs (numpy; identical on any host).

splitmix64(seed, i) -> uniform / normal / int draws.  Normals use Box-Muller in
float64 and are rounded to the target dtype (f32 RNE, then bf16 RNE).
"""
import numpy as np

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SEED_BASE = 0x48465553494F4E01  # "HFUSION\x01"


def splitmix64(seed, n, offset=0):
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(offset, offset + n, dtype=np.uint64) + np.uint64(1)) * _G
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_f32(seed, shape, lo, hi):
    n = int(np.prod(shape))
    u = (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal_f64(seed, n):
    z1 = splitmix64(seed, n)
    z2 = splitmix64(seed ^ 0x5DEECE66D, n)
    u1 = ((z1 >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / (1 << 53))
    u2 = (z2 >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def normal_f32(seed, shape, std=1.0):
    n = int(np.prod(shape))
    return (normal_f64(seed, n) * std).astype(np.float32).reshape(shape)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(seed, shape, std=1.0):
    return f32_to_bf16_bits(normal_f32(seed, shape, std)).reshape(shape)


def uniform_bf16(seed, shape, lo, hi):
    return f32_to_bf16_bits(uniform_f32(seed, shape, lo, hi)).reshape(shape)


def int8_uniform(seed, shape, lo=-127, hi=127):
    n = int(np.prod(shape))
    z = splitmix64(seed, n) % np.uint64(hi - lo + 1)
    return (z.astype(np.int64) + lo).astype(np.int8).reshape(shape)


def argmax_logits(seed, rows, cols, dup_every=100):
    """N(0,1) logits; rows r % dup_every == 0 get their maximum copied to 2-3
    other positions before and after the original argmax (lowest-index tie
    break)."""
    x = normal_f32(seed, (rows, cols))
    for r in range(0, rows, dup_every):
        j = int(np.argmax(x[r]))
        m = x[r, j]
        z = splitmix64(seed + 7 + r, 4)
        k = 2 + int(z[0] % np.uint64(2))
        for t in range(k):
            pos = int(z[1 + t % 3] % np.uint64(cols))
            if t == 0 and j > 0:
                pos = int(z[1] % np.uint64(j))  # one copy strictly before
            x[r, pos] = m
    return x


def config_inputs(name, **kw):
    """Inputs of the headline configuration `name` (seed SEED_BASE + index)."""
    if name == "vec_add":
        n = kw.get("n", 1 << 24)
        s = SEED_BASE + 0
        return [uniform_f32(s, (n,), -1.0, 1.0), uniform_f32(s + 1, (n,), -1.0, 1.0)]
    if name == "rmsnorm_quant":
        r, c = kw.get("rows", 8192), kw.get("cols", 4096)
        s = SEED_BASE + 1
        return [normal_bf16(s, (r, c)), uniform_bf16(s + 1, (c,), 0.5, 1.5)]
    if name == "safe_softmax":
        r, c = kw.get("rows", 4096), kw.get("cols", 32768)
        return [normal_f32(SEED_BASE + 2, (r, c), std=2.0)]
    if name == "argmax":
        r, c = kw.get("rows", 256), kw.get("cols", 152064)
        return [argmax_logits(SEED_BASE + 3, r, c)]
    if name == "w8a8_dequant":
        m, n, k = kw.get("m", 4096), kw.get("n", 4096), kw.get("k", 4096)
        s = SEED_BASE + 4
        return [int8_uniform(s, (m, k)), int8_uniform(s + 1, (n, k)),
                uniform_f32(s + 2, (m,), 0.001, 0.02), uniform_f32(s + 3, (n,), 0.001, 0.02)]
    raise KeyError(name)
