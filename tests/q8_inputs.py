"""Activation generators shared by the CPU and GPU quantization tests."""
import numpy as np


def near_tie_rows(m: int, k: int, seed: int) -> np.ndarray:
    """Blocks whose quotients x / d sit on, or within 2 ulp of, half-integers.

    The kernels round x * (1 / d) and fall back to the division only near a
    tie; these values are where a wrong window would pick the other integer.
    Block maxima span 1e-44 (d subnormal or zero) to 1e38. Value 0 of each
    block is its amax, so d = f32(amax / 127) is known here; the rest are
    f32((n + 1/2) * d) moved by -2..2 ulp, clipped to amax.
    """
    rng = np.random.default_rng(seed)
    nb = m * k // 32
    amax = (np.float32(10.0) ** rng.uniform(-44, 38, nb).astype(np.float32)).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    n = rng.integers(-127, 127, (nb, 31)).astype(np.float32)
    v = ((n + np.float32(0.5)) * d[:, None]).astype(np.float32)
    steps = rng.integers(-2, 3, (nb, 31))
    for s in (1, 2):
        v = np.where(steps >= s, np.nextafter(v, np.float32(np.inf)), v)
        v = np.where(steps <= -s, np.nextafter(v, np.float32(-np.inf)), v)
    v = np.clip(v, -amax[:, None], amax[:, None]).astype(np.float32)
    return np.concatenate([amax[:, None], v], axis=1).reshape(m, k).astype(np.float32)


def s16_tie_blocks(nblocks: int, seed: int) -> np.ndarray:
    """Blocks whose Q8_1 sum field is an f16 rounding tie after the f32 product.

    s16 = f16(f32(d * S)) rounds twice. When f32(d * S) lands exactly halfway
    between two f16 values while the exact product d * S does not, rounding
    the exact product once (a fused multiply-convert) picks the other f16
    value. Returns [nblocks, 32] f32 blocks (searched among N(0, 1) blocks
    with numpy's IEEE float32 arithmetic) where the two roundings differ.
    """
    rng = np.random.default_rng(seed)
    found = []
    while sum(len(f) for f in found) < nblocks:
        x = rng.standard_normal((1 << 18, 32)).astype(np.float32)
        amax = np.max(np.abs(x), axis=1)
        d = (amax / np.float32(127.0)).astype(np.float32)
        q = np.rint(x / d[:, None]).astype(np.float32)
        S = np.sum(q, axis=1, dtype=np.float64).astype(np.float32)
        twice = (d * S).astype(np.float32).astype(np.float16)
        once = (d.astype(np.float64) * S.astype(np.float64)).astype(np.float16)
        found.append(x[twice != once])
    return np.concatenate(found)[:nblocks]
