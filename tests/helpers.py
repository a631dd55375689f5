"""Input generators shared by the tests.

`fill` and `labels` restate the reference test helpers bit-for-bit
(tests/end_to_end.rs:14-36): a 64-bit LCG giving uniforms in [-scale, scale)
and labels `(i*7+3) % V` with every k-th row ignored.
"""
import numpy as np

M64 = (1 << 64) - 1


def fill(n: int, seed: int, scale: float) -> np.ndarray:
    """tests/end_to_end.rs:14-27 (the f32 arithmetic is reproduced exactly)."""
    s = (seed * 2862933555777941757 + 3037000493) & M64
    out = np.empty(n, np.float32)
    two31 = np.float32(1 << 31)
    two = np.float32(2.0)
    one = np.float32(1.0)
    sc = np.float32(scale)
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & M64
        u = np.float32(s >> 33) / two31
        out[i] = (u * two - one) * sc
    return out


def mat(rows: int, cols: int, seed: int, scale: float) -> np.ndarray:
    return fill(rows * cols, seed, scale).reshape(rows, cols)


def labels(bt: int, v: int, ignore_every=None, ignore_index: int = -100) -> np.ndarray:
    """tests/end_to_end.rs:29-36"""
    out = np.empty(bt, np.int64)
    for i in range(bt):
        if ignore_every is not None and i % ignore_every == 0:
            out[i] = ignore_index
        else:
            out[i] = (i * 7 + 3) % v
    return out


def normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """Seeded N(0, std^2) float32 matrix (numpy PCG64)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def uniform_labels(bt: int, v: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, v, size=bt, dtype=np.int64)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) >> 16) << 16
    nan = np.isnan(a)
    out = r.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out
