"""CPU restatement of block-sparse softmax attention.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

Semantics of SpargeAttn's block-sparse kernel
(``csrc/qattn/qk_int_sv_f16_cuda_sm80.cuh:42-738`` inside
``third_party/spargeattn.zip``): query block ``i`` (``block_q`` rows) attends
to the union of its listed ``block_k``-key blocks; keys at or beyond the
sequence end are excluded (the kernel masks them to -5e6 on the final block,
``.cuh:585``); softmax is exact (base-2 online softmax is an implementation
detail); rows beyond the query end are not written. The reference kernel
quantises Q/K to int8 and P to fp16; this oracle is the exact float64
computation that both the reference and the bf16 HIP kernel approximate.

Pinning: ``tests/test_oracle_misc.py`` checks it against
``torch.nn.functional.scaled_dot_product_attention`` with a dense boolean
mask in float64, and that full index lists reproduce dense attention.
``pv_post_cut`` (the PV threshold) is pinned by hand-computed decision
sequences on rank-one logits, the strict ``gap + threshold > 0`` boundary,
the inert 1e10 threshold and the zero logits of padded query rows.
"""
from __future__ import annotations

import math

import numpy as np


def block_sparse_attention(q, k, v, index_lists, counts, *, block_q: int = 128,
                           block_k: int = 64, scale: float | None = None, q_blocks=None) -> np.ndarray:
    """float64 attention of ``q [B,H,Nq,D]`` over listed key blocks.

    ``index_lists [B,H,Qb,W]`` absolute key-block indices (entries past
    ``counts`` ignored). Rows with a zero count produce zeros.
    ``q_blocks`` (optional): only these query blocks are computed, the rows
    of the others stay zero (sampled checks of long sequences).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, Nq, D = q.shape
    Tk = k.shape[-2]
    scale = D ** -0.5 if scale is None else scale
    Qb = -(-Nq // block_q)
    out = np.zeros((B, H, Nq, v.shape[-1]), np.float64)
    blocks_to_do = range(Qb) if q_blocks is None else sorted({int(i) for i in q_blocks})
    for b in range(B):
        for h in range(H):
            for i in blocks_to_do:
                n = int(counts[b, h, i])
                if n == 0:
                    continue
                blocks = np.asarray(index_lists[b, h, i, :n], np.int64)
                keys = (blocks[:, None] * block_k + np.arange(block_k)[None]).reshape(-1)
                keys = keys[keys < Tk]
                rows = slice(i * block_q, min((i + 1) * block_q, Nq))
                s = q[b, h, rows] @ k[b, h, keys].T * scale
                s = s - s.max(axis=-1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=-1, keepdims=True)
                out[b, h, rows] = p @ v[b, h, keys]
    return out


def pv_post_cut(q, k, index_lists, counts, pv_threshold, *, block_q: int = 128, block_k: int = 64,
                scale: float | None = None, waves: int = 4):
    """The PV post-cut's decisions (qk_int_sv_f16_cuda_sm80.cuh:291-381 with
    update_mo, attn_utils.cuh:419-466, per-block mode).

    For each query block, over its listed key blocks in list order: the
    block row max ``max(-5e6, max_key logit) * scale * log2 e`` (query rows
    past ``Nq`` count with zero logits), gap = max over the block's rows of
    (block row max - running row max), running max (from -5e6) raised to the
    block row max whether or not PV runs. PV runs when gap + threshold > 0.

    Returns ``(lists, counts, pv_map)``: the executed blocks (list order) and
    the int32 map ``[B, H, Qb*waves, Kb]`` with 1 where each query wave ran
    PV. Attention over the executed lists (``block_sparse_attention``) is the
    post-cut output: a skipped block adds to neither numerator nor sum.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, H, Nq, D = q.shape
    Tk = k.shape[-2]
    Kb = -(-Tk // block_k)
    scale = D ** -0.5 if scale is None else scale
    c = scale * math.log2(math.e)
    thr = np.broadcast_to(np.asarray(pv_threshold, np.float64).reshape(-1), (H,))
    Qb = -(-Nq // block_q)
    W = index_lists.shape[-1]
    lists = np.full((B, H, Qb, W), -1, np.int32)
    cnt = np.zeros((B, H, Qb), np.int32)
    pv_map = np.zeros((B, H, Qb * waves, Kb), np.int32)
    for b in range(B):
        for h in range(H):
            for i in range(Qb):
                rows = np.zeros((block_q, D))
                r1 = min((i + 1) * block_q, Nq)
                rows[: r1 - i * block_q] = q[b, h, i * block_q: r1]
                run = np.full(block_q, -5e6)
                for blk in np.asarray(index_lists[b, h, i, : int(counts[b, h, i])], np.int64):
                    keys = blk * block_k + np.arange(block_k)
                    keys = keys[keys < Tk]
                    bm = np.maximum(-5e6, (rows @ k[b, h, keys].T).max(axis=-1)) * c
                    gap = (bm - run).max()
                    run = np.maximum(run, bm)
                    if gap + thr[h] > 0:
                        lists[b, h, i, cnt[b, h, i]] = blk
                        cnt[b, h, i] += 1
                        pv_map[b, h, i * waves:(i + 1) * waves, blk] = 1
    return lists, cnt, pv_map


def dense_lists(B: int, H: int, Nq: int, Tk: int, block_q: int = 128, block_k: int = 64):
    """Index lists that name every key block for every query block."""
    Qb = -(-Nq // block_q)
    nk = -(-Tk // block_k)
    lists = np.broadcast_to(np.arange(nk, dtype=np.int32), (B, H, Qb, nk)).copy()
    counts = np.full((B, H, Qb), nk, dtype=np.int32)
    return lists, counts
