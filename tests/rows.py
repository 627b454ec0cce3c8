"""Random GGUF rows of every format with finite fp16 scales (test inputs)."""
import numpy as np

BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 14: (256, 210)}


def row_bytes(t: int, k: int) -> int:
    e, b = BLOCK[t]
    return k // e * b


def _f16(rng, n, scale):
    return (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint8).reshape(n, 2)


def random_rows(rng, t: int, k: int, n: int) -> np.ndarray:
    """n GGUF rows of type t and length k: random quant bytes, finite fp16 scales."""
    if t == 0:
        return (rng.standard_normal((n, k)).astype(np.float32) * 0.05).view(np.uint8).reshape(n, k * 4)
    if t == 1:
        return (rng.standard_normal((n, k)) * 0.05).astype(np.float16).view(np.uint8).reshape(n, k * 2)
    e, b = BLOCK[t]
    nb = n * (k // e)
    blk = rng.integers(0, 256, size=(nb, b), dtype=np.uint8)
    if t == 8:
        blk[:, 0:2] = _f16(rng, nb, 0.001)
    elif t == 2:
        blk[:, 0:2] = _f16(rng, nb, 0.005)
    elif t == 3:
        blk[:, 0:2] = _f16(rng, nb, 0.005)
        blk[:, 2:4] = _f16(rng, nb, 0.02)
    elif t == 14:
        blk[:, 208:210] = _f16(rng, nb, 0.0005)
    return blk.reshape(n, (k // e) * b)


