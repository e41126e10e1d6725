"""Shared test helpers: block builders, seeded inputs and the parity bound."""
from __future__ import annotations

import numpy as np

Q8_0 = 1
Q4_0 = 2
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

# Per-config seeds (BASELINE.json says "fixed seed" without a value):
# SEED_BASE + config index.
SEED_BASE = 20261201


def q8_blocks(scales, values) -> np.ndarray:
    """Q8_0 bytes from per-block fp16 scale bits and int8 values [nblocks, 32]."""
    scales = np.asarray(scales, np.uint16).reshape(-1)
    values = np.asarray(values).reshape(-1, 32)
    out = np.empty((scales.size, 34), np.uint8)
    out[:, 0:2] = scales.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = values.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def q4_blocks(scales, nibbles) -> np.ndarray:
    """Q4_0 bytes from fp16 scale bits and packed nibble bytes [nblocks, 16]."""
    scales = np.asarray(scales, np.uint16).reshape(-1)
    nibbles = np.asarray(nibbles, np.uint8).reshape(-1, 16)
    out = np.empty((scales.size, 18), np.uint8)
    out[:, 0:2] = scales.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = nibbles
    return out.reshape(-1)


def random_blocks(rng: np.random.Generator, type_: int, rows: int, cols: int, scale_bits=None) -> np.ndarray:
    """Random quantised matrix; scales from `scale_bits` (cycled) or random normal fp16."""
    nb = rows * cols // 32
    if scale_bits is None:
        scales = rng.normal(0.0, 0.02, nb).astype(np.float16).view(np.uint16)
    else:
        scale_bits = np.asarray(scale_bits, np.uint16)
        scales = scale_bits[np.arange(nb) % scale_bits.size]
    if type_ == Q8_0:
        return q8_blocks(scales, rng.integers(-128, 128, (nb, 32)))
    return q4_blocks(scales, rng.integers(0, 256, (nb, 16)))


def dequant_numpy(w: np.ndarray, type_: int, rows: int, cols: int) -> np.ndarray:
    """Independent numpy dequantisation (q8.h / q4.h layouts) for norms and bounds."""
    nb = rows * cols // 32
    blk = w.reshape(nb, BLOCK_BYTES[type_])
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nb, 1)
    if type_ == Q8_0:
        q = blk[:, 2:].view(np.int8).astype(np.float32)
    else:
        nib = blk[:, 2:]
        q = np.concatenate([(nib & 15).astype(np.float32) - 8, (nib >> 4).astype(np.float32) - 8], axis=1)
    return (d * q).reshape(rows, cols)


def row_bound(wd: np.ndarray, x: np.ndarray, factor: float = 1e-5) -> np.ndarray:
    """max|delta| allowed per output: factor * ||w_row||_2 * ||x||_2 (double)."""
    wn = np.sqrt(np.sum(np.square(wd.astype(np.float64)), axis=1))
    xn = np.sqrt(np.sum(np.square(np.asarray(x, np.float64)), axis=-1))
    if np.ndim(xn) == 0:
        return factor * wn * xn
    return factor * xn[:, None] * wn[None, :]


def lcg_sampler(seed: int = 42):
    """The reference tests' LCG (tests/q8_cpu_test.cpp:59-63): values in [-1, 1)."""
    state = [seed & 0xFFFFFFFF]

    def sample() -> np.float32:
        state[0] = (state[0] * 1664525 + 1013904223) & 0xFFFFFFFF
        return np.float32((int(state[0] >> 16) - 32768) / 32768.0)

    return sample


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
