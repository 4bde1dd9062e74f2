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


def pooled_logits(pooled_q: np.ndarray, pooled_k: np.ndarray, *, bf16: bool = True,
                  scale: float | None = None) -> np.ndarray:
    """Scaled pooled logits ``[..., Qb, Kb]`` in float32 (scale ``1/sqrt(d)`` by default)."""
    d = pooled_q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
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


def bf16_spacing(x) -> np.ndarray:
    """Gap between consecutive bfloat16 values at ``|x|``: ``2^(e-7)`` for
    ``|x|`` in ``[2^e, 2^(e+1))`` (the normal range's smallest gap below it).
    Two roundings of values ``a``, ``b`` to bfloat16 differ by at most
    ``|a - b| + bf16_spacing(max(|a|, |b|))``."""
    a = np.abs(np.asarray(x, np.float64))
    return np.exp2(np.floor(np.log2(np.maximum(a, 2.0 ** -126))) - 7)


def logit_error_bound(pooled_q: np.ndarray, pooled_k: np.ndarray, scale: float | None = None, *,
                      bf16: bool = True) -> np.ndarray:
    """Largest difference ``[..., Qb, Kb]`` between this oracle's logits and
    those of any kernel that sums the 64 exact bf16 products in float32 in
    any order, then applies the same roundings.

    The float32 sum is within ``63 * 2^-24 * sum|q_d k_d|`` of the exact dot
    product; this oracle's float64 sum rounded to float32 is within
    ``2^-24 |dot|``; with ``bf16`` both are then rounded to bfloat16 (one
    ``bf16_spacing`` at most), multiplied by the scale and rounded again (exact
    for a power-of-two scale, one more spacing otherwise).
    """
    q = np.asarray(pooled_q, np.float64)
    k = np.asarray(pooled_k, np.float64)
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    dot = np.einsum("...qd,...kd->...qk", q, k)
    mag = np.einsum("...qd,...kd->...qk", np.abs(q), np.abs(k))
    err = (d - 1) * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(dot)
    if bf16:
        err = err + bf16_spacing(np.abs(dot) + err)
        err = err * abs(scale)
        if math.frexp(abs(scale))[0] != 0.5:
            err = err + bf16_spacing(np.abs(dot * scale) + err)
        return err
    return err * abs(scale) + 2.0 ** -24 * np.abs(dot * scale)


def prob_error_bound(prob_ref: np.ndarray, logit_err: np.ndarray, logits: np.ndarray, *,
                     fp32_rel: float = 2e-5) -> np.ndarray:
    """Element-wise bound on ``|p - prob_ref|`` for a softmax whose logits
    are each within ``logit_err`` of the reference's.

    ``log p_j`` moves by the logit's own change plus the change of the row's
    log-sum-exp, which is a probability-weighted mean of the logit changes
    (``sum_k p'_k delta_k`` at an intermediate point, where ``p'_k <=
    p_k * exp(2 max delta)``), so at most ``min(max delta, exp(2 max delta) *
    sum_k p_k delta_k)``. ``fp32_rel`` plus 16 float32 spacings of the row's
    largest logit cover the kernel's own float32 exponentials and sum; the
    2e-38 floor covers probabilities below float32's normal range.
    """
    p = np.asarray(prob_ref, np.float64)
    e = np.asarray(logit_err, np.float64)
    emax = e.max(axis=-1, keepdims=True)
    lse = np.minimum(emax, np.exp(2 * emax) * (p * e).sum(axis=-1, keepdims=True))
    big = np.abs(np.asarray(logits, np.float32)).max(axis=-1, keepdims=True)
    rel = fp32_rel + 16 * np.spacing(big).astype(np.float64)
    return p * np.expm1(e + lse + rel) + 2e-38


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


def prob_outside_bound(got: np.ndarray, pooled_q: np.ndarray, pooled_k: np.ndarray, scale: float | None = None,
                       *, bf16: bool = True) -> np.ndarray:
    """Boolean map of the entries of a kernel's pooled probabilities ``got``
    that lie outside ``prob_error_bound`` around this oracle's softmax of the
    same pooled means (an empty map, ``.any()`` false, is the pass)."""
    q = np.asarray(pooled_q, np.float32)
    k = np.asarray(pooled_k, np.float32)
    logits = pooled_logits(q, k, bf16=bf16, scale=scale)
    ref = softmax(logits)
    bound = prob_error_bound(ref, logit_error_bound(q, k, scale, bf16=bf16), logits)
    return np.abs(np.asarray(got, np.float64) - ref.astype(np.float64)) > bound
