"""Seeded synthetic inputs of the shapes and distributions the benchmark configs name.

All generators are numpy-only and deterministic for a given seed.
  fp8_weight      uniform e4m3fn bytes with the NaN codes (0x7F, 0xFF) redrawn
  fp8_scales      fp32 per 128x128 block, log-uniform in [1e-3, 1e-1]
  q4k_blocks      144-byte super-blocks: fp16 d/dmin in [1e-4, 1e-2], random
                  6-bit scales/mins (12 random bytes), random nibbles
  q6k_blocks      210-byte super-blocks: random ql/qh, int8 scales, fp16 d
"""
from __future__ import annotations

import numpy as np

NAN_CODES = (0x7F, 0xFF)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def fp8_weight(r: np.random.Generator, m: int, n: int) -> np.ndarray:
    w = r.integers(0, 256, size=(m, n), dtype=np.uint8)
    bad = (w == 0x7F) | (w == 0xFF)
    while bad.any():
        w[bad] = r.integers(0, 256, size=int(bad.sum()), dtype=np.uint8)
        bad = (w == 0x7F) | (w == 0xFF)
    return w


def fp8_scales(r: np.random.Generator, m: int, n: int, lo=1e-3, hi=1e-1) -> np.ndarray:
    shape = ((m + 127) // 128, (n + 127) // 128)
    return np.exp(r.uniform(np.log(lo), np.log(hi), size=shape)).astype(np.float32)


def _fp16_bits(r: np.random.Generator, count: int, lo: float, hi: float) -> np.ndarray:
    return r.uniform(lo, hi, size=count).astype(np.float16).view(np.uint16)


def q4k_blocks(r: np.random.Generator, m: int, n: int) -> np.ndarray:
    """[m][n/256 * 144] uint8 (row-major rows of Q4_K super-blocks)."""
    assert n % 256 == 0
    nb = m * (n // 256)
    blk = np.empty((nb, 144), np.uint8)
    blk[:, 0:2] = _fp16_bits(r, nb, 1e-4, 1e-2).view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = _fp16_bits(r, nb, 1e-4, 1e-2).view(np.uint8).reshape(nb, 2)
    blk[:, 4:144] = r.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    return blk.reshape(m, -1)


def q6k_blocks(r: np.random.Generator, m: int, n: int) -> np.ndarray:
    """[m][n/256 * 210] uint8 (row-major rows of Q6_K super-blocks)."""
    assert n % 256 == 0
    nb = m * (n // 256)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, 0:208] = r.integers(0, 256, size=(nb, 208), dtype=np.uint8)
    blk[:, 208:210] = _fp16_bits(r, nb, 1e-4, 1e-2).view(np.uint8).reshape(nb, 2)
    return blk.reshape(m, -1)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns with round-to-nearest-even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def fp8_weight_wide(r: np.random.Generator, m: int, n: int) -> np.ndarray:
    """Uniform over the 254 finite e4m3fn codes in one pass (codes >= 0x7F shifted
    past the NaN code 0x7F; 0xFE stays the top): for matrices of the full model
    width, where redrawing NaN codes costs several passes."""
    w = r.integers(0, 254, size=(m, n), dtype=np.uint8)
    w += (w >= 0x7F).view(np.uint8)
    return w


def bf16_random_bits(r: np.random.Generator, m: int, n: int) -> np.ndarray:
    """Random bf16 values of magnitude (1 + f) * 2^e, e in -8..-5 (about 0.004 to
    0.03), random sign and mantissa, built from one uint16 draw per entry: for
    vocabulary-sized tables (a normal draw of 1.3G entries takes minutes)."""
    words = (m * n + 3) // 4
    u = r.integers(0, np.iinfo(np.uint64).max, size=words, dtype=np.uint64, endpoint=True)
    u = u.view(np.uint16)[: m * n].reshape(m, n)
    # sign and mantissa kept, exponent field = 119 + (two random bits 7-8)
    out = u & np.uint16(0x81FF)
    out += np.uint16((127 - 8) << 7)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)
