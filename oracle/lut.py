"""CPU restatement of SpargeAttn's block-map LUT.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

``encode`` follows ``triton_block_map_to_lut_kernel``
(``spas_sage_attn/utils.py:54-87`` inside ``third_party/spargeattn.zip``):
for each row the selected columns in ascending order, stored as deltas (the
first entry absolute), zero-filled, plus the count. ``decode`` inverts it.

Pinning: ``tests/test_oracle_misc.py`` checks ``encode`` against an
independent restatement of the reference's torch ``block_map_lut``
(``utils.py:417-430``: cumsum, sort, difference) and checks
``decode(encode(m)) == m`` on random maps including empty and full rows.
"""
from __future__ import annotations

import numpy as np


def encode(block_map: np.ndarray):
    """Bool ``[..., K]`` -> (int32 delta LUT ``[..., K]``, int32 counts)."""
    m = np.asarray(block_map, dtype=bool)
    K = m.shape[-1]
    flat = m.reshape(-1, K)
    lut = np.zeros(flat.shape, dtype=np.int32)
    cnt = np.zeros(flat.shape[0], dtype=np.int32)
    for r in range(flat.shape[0]):
        nz = np.flatnonzero(flat[r])
        if nz.size:
            lut[r, : nz.size] = np.diff(nz, prepend=0)
        cnt[r] = nz.size
    return lut.reshape(m.shape), cnt.reshape(m.shape[:-1])


def decode(lut: np.ndarray, counts: np.ndarray, K: int | None = None) -> np.ndarray:
    """Inverse of ``encode``."""
    lut = np.asarray(lut, dtype=np.int64)
    K = lut.shape[-1] if K is None else K
    flat = lut.reshape(-1, lut.shape[-1])
    c = np.asarray(counts).reshape(-1)
    out = np.zeros((flat.shape[0], K), dtype=bool)
    for r in range(flat.shape[0]):
        idx = np.cumsum(flat[r, : c[r]])
        out[r, idx] = True
    return out.reshape(lut.shape[:-1] + (K,))


def reference_block_map_lut(block_map: np.ndarray):
    """Independent restatement of ``block_map_lut`` (utils.py:417-430)."""
    m = np.asarray(block_map, dtype=bool)
    valid = m.astype(np.int32).sum(-1)
    cum = np.cumsum(np.ones(m.shape, dtype=np.int64), axis=-1) * m
    filled = np.where(m, cum, 10000000)
    lut = np.sort(filled, axis=-1) - 1
    lut[..., 1:] = lut[..., 1:] - lut[..., :-1]
    return lut.astype(np.int32), valid.astype(np.int32)
