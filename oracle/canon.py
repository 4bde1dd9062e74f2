"""Canonical reductions shared bit-for-bit by the oracle and the HIP kernels.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

The reference computes its selector sums with torch's fp32 reductions, whose
order is an implementation detail (``SW:1765, 3788-3791, 3837-3839, 3854``;
``SW`` = ``src/sparse_vggt/utils/sparse_wrapper.py``). To make block-index
lists reproducible bit-for-bit between this oracle and the GPU, every sum on
the selection path is defined here with a fixed order and float64
accumulation, rounded once to float32 where the reference holds a float32
tensor. The HIP select kernels implement exactly these orders.

``wave_sum``   lane j (0..63) accumulates x[j], x[j+64], x[j+128], ... in
               float64 in increasing index order starting from +0.0, then an
               xor butterfly over offsets 32, 16, 8, 4, 2, 1 combines the 64
               lane sums (``s_j = s_j + s_{j^o}``). IEEE addition is
               commutative, so every lane ends with the same value.
``seq_sum``    float64, strictly sequential in index order from +0.0.
``chunked_sum`` float64: ``seq_sum`` inside consecutive chunks of ``CHUNK``
               (32) elements, then ``seq_sum`` over the chunk partials.

Pinning: ``tests/test_oracle_canon.py`` checks both against exact rational
sums (``fractions.Fraction``) on inputs whose float64 sums are exact, against
a scalar re-implementation of the lane/butterfly loop, and that a plausible
mistake (a missing butterfly stage, a reversed order on inputs where order
matters) changes the result.
"""
from __future__ import annotations

import numpy as np

WAVE = 64
FLT_MAX = np.float32(np.finfo(np.float32).max)
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def f32(x):
    """Round to float32 (round-to-nearest-even)."""
    return np.asarray(x, dtype=np.float64).astype(np.float32)


def wave_sum(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Canonical 64-lane tree sum in float64 along ``axis``.

    Returns float64 with ``axis`` removed.
    """
    x = np.moveaxis(np.asarray(x), axis, -1).astype(np.float64)
    n = x.shape[-1]
    lanes = np.zeros(x.shape[:-1] + (WAVE,), dtype=np.float64)
    for start in range(0, n, WAVE):
        chunk = x[..., start:start + WAVE]
        width = chunk.shape[-1]
        lanes[..., :width] = lanes[..., :width] + chunk
    idx = np.arange(WAVE)
    for off in (32, 16, 8, 4, 2, 1):
        lanes = lanes + lanes[..., idx ^ off]
    return lanes[..., 0].copy()


def seq_sum(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Strictly sequential float64 sum along ``axis`` (returns float64)."""
    x = np.moveaxis(np.asarray(x), axis, -1).astype(np.float64)
    acc = np.zeros(x.shape[:-1], dtype=np.float64)
    for i in range(x.shape[-1]):
        acc = acc + x[..., i]
    return acc


CHUNK = 32


def chunked_sum(x: np.ndarray, axis: int = -1, chunk: int = CHUNK) -> np.ndarray:
    """Sequential float64 sums of ``chunk``-element chunks, then sequential
    over the partials (returns float64)."""
    x = np.moveaxis(np.asarray(x), axis, -1).astype(np.float64)
    n = x.shape[-1]
    total = np.zeros(x.shape[:-1], dtype=np.float64)
    for start in range(0, n, chunk):
        total = total + seq_sum(x[..., start:start + chunk], axis=-1)
    return total


def clamp01(x: np.ndarray) -> np.ndarray:
    """``clamp(x, 0, 1)`` with torch's NaN propagation, in float32."""
    x = np.asarray(x, dtype=np.float32)
    out = np.where(x < 0, np.float32(0.0), x)
    out = np.where(out > 1, np.float32(1.0), out)
    return out.astype(np.float32)


def clamp_min0(x: np.ndarray) -> np.ndarray:
    """``clamp_min(x, 0)`` with NaN propagation; ``-0.0`` becomes ``+0.0``."""
    x = np.asarray(x, dtype=np.float32)
    return np.where(x > 0, x, np.where(np.isnan(x), x, np.float32(0.0))).astype(np.float32)


def order_key(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of float32 values (descending selection).

    ``-0.0`` is folded onto ``+0.0``; NaN (positive quiet) sorts above
    ``+inf`` which mirrors torch's descending sort/topk placing NaN first.
    """
    x = np.asarray(x, dtype=np.float32)
    x = np.where(x == 0, np.float32(0.0), x)
    x = np.where(np.isnan(x), np.float32(np.nan), x)
    bits = x.view(np.uint32).astype(np.uint64)
    neg = (bits >> 31) & 1
    key = np.where(neg == 1, bits ^ 0xFFFFFFFF, bits ^ 0x80000000)
    return key.astype(np.uint32)
