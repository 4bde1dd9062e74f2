"""CPU restatement of block pooling and the pooled-score predictor.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

* ``pool_blocks``   ``F.avg_pool1d(kernel, ceil_mode=True)`` over tokens as
                    used by ``predict_attention`` (``ATT:60-68``, ``ATT`` =
                    ``src/sparse_vggt/models/attention.py``) and
                    ``_mean_pool_contiguous_value_blocks`` (``SW:2839-2861``):
                    each full block is the mean of its tokens, the tail block
                    the mean of its real tokens only.
* ``pooled_prob``   ``softmax(pooled_q @ pooled_k^T / sqrt(d))`` (``ATT:97-101``)
                    with the roundings the reference incurs under bf16 autocast
                    when ``bf16=True``: pooled means rounded to bf16, logits
                    rounded to bf16 by the bf16 matmul, the scale multiply
                    rounded to bf16, softmax in fp32 (autocast promotes it).

Parity pins: ``tests/test_oracle_misc.py`` checks the pooling against
brute-force per-block means (exact rational arithmetic on small cases) and
against ``torch.nn.functional.avg_pool1d(ceil_mode=True)``; the predictor
against golden vectors from the reference's ``predict_attention`` run on CPU in
bf16 (``tests/golden/make_golden.py``) and against a float64 softmax.
"""
from __future__ import annotations

import math

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (RNE), returned as float32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = x.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    out = rounded.view(np.float32).copy()
    out[nan] = np.float32(np.nan)
    return out


def pool_blocks(x: np.ndarray, block: int, *, round_bf16: bool = False) -> np.ndarray:
    """Mean over consecutive ``block`` tokens of ``x [..., T, D]``.

    The tail block averages only its real tokens. Sums are float64; the mean
    is rounded to float32 (and to bf16 when ``round_bf16``).
    """
    x = np.asarray(x, dtype=np.float64)
    T = x.shape[-2]
    nb = math.ceil(T / block)
    out = np.empty(x.shape[:-2] + (nb, x.shape[-1]), dtype=np.float64)
    for i in range(nb):
        seg = x[..., i * block:min((i + 1) * block, T), :]
        out[..., i, :] = seg.sum(axis=-2) / seg.shape[-2]
    if round_bf16:
        return bf16_round(out.astype(np.float32))
    return out.astype(np.float32)


def max_pool_blocks(x: np.ndarray, block: int) -> np.ndarray:
    """``F.max_pool1d(kernel_size=block, ceil_mode=True)`` over the tokens of
    ``x [..., T, D]``: the tail block takes the max of its real tokens (the
    max of bf16 values is itself a bf16 value, so no rounding)."""
    x = np.asarray(x, dtype=np.float32)
    T = x.shape[-2]
    nb = math.ceil(T / block)
    out = np.empty(x.shape[:-2] + (nb, x.shape[-1]), dtype=np.float32)
    for i in range(nb):
        out[..., i, :] = x[..., i * block:min((i + 1) * block, T), :].max(axis=-2)
    return out


def pooled_logits(pooled_q: np.ndarray, pooled_k: np.ndarray, *, bf16: bool = True) -> np.ndarray:
    """Scaled pooled logits ``[..., Qb, Kb]`` in float32."""
    d = pooled_q.shape[-1]
    scale = 1.0 / math.sqrt(d)
    dots = np.einsum("...qd,...kd->...qk", pooled_q.astype(np.float64), pooled_k.astype(np.float64))
    if bf16:
        dots = bf16_round(dots.astype(np.float32))
        return bf16_round((dots * np.float32(scale)).astype(np.float32))
    return (dots * scale).astype(np.float32)


def softmax(logits: np.ndarray) -> np.ndarray:
    """Row softmax in float64, rounded to float32."""
    z = np.asarray(logits, dtype=np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def pooled_prob(q: np.ndarray, k: np.ndarray, ks_q: int = 128, ks_k: int = 64, *, bf16: bool = True,
                pool_mode: str = "avg"):
    """``predict_attention(q, k, ks_q, ks_k, pool_mode)`` (ATT:31-104).

    Returns ``(prob [B,H,Qb,Kb] float32, pooled_q, pooled_k)``.
    """
    if pool_mode == "max":
        pq, pk = max_pool_blocks(q, ks_q), max_pool_blocks(k, ks_k)
    else:
        pq = pool_blocks(q, ks_q, round_bf16=bf16)
        pk = pool_blocks(k, ks_k, round_bf16=bf16)
    return softmax(pooled_logits(pq, pk, bf16=bf16)), pq, pk


def key_block_variance(k: np.ndarray, ks_k: int = 64, *, bf16: bool = True) -> np.ndarray:
    """``predict_attention(..., return_key_block_variance=True)``'s second
    output (ATT:69-89): per 64-key block, the mean over its real tokens of
    the squared token norm minus the squared norm of the block mean, clamped
    at 0, ``[B,H,Kb]`` float32. With ``bf16`` the token squares are rounded to
    bfloat16 before their float32 sum (``key * key`` on bf16 keys) and the
    block mean is the bf16-rounded mean, as under bf16 autocast."""
    k = np.asarray(k, np.float32)
    sq = (k * k).astype(np.float32)
    if bf16:
        sq = bf16_round(sq)
    tok = sq.astype(np.float64).sum(-1).astype(np.float32)                  # [B,H,T]
    mean_sq = pool_blocks(tok[..., None], ks_k)[..., 0]                      # float32 block means
    mean = pool_blocks(k, ks_k, round_bf16=bf16)                             # [B,H,Kb,D]
    sq_mean = (mean.astype(np.float64) ** 2).sum(-1).astype(np.float32)
    return np.maximum((mean_sq - sq_mean).astype(np.float32), np.float32(0.0))
