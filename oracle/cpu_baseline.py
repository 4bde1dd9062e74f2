"""PyTorch-CPU fp32 restatement of the reference's dense and Top-K
global-attention ops.

TEST/BENCH INFRASTRUCTURE (see ``oracle/__init__.py``): used only by the
``cpu_baseline`` leg of ``bench.py`` as the reported CPU figure.

* ``topk_layer``: one layer of the reference's ``topk`` path on the CPU:
  pooled predictor (``attention.py:31-104``), per-row Top-K over key blocks
  plus sink blocks (``sparse_wrapper.py:1199-1268``), then softmax attention
  of each 128-query block over the keys of its kept 64-key blocks (the
  semantics of ``qk_int_sv_f16_cuda_sm80.cuh``);
* ``dense_layer``: the ``dense`` mode's attention (the unpatched upstream
  layer's SDPA over every key, ``evaluate.py:193-195``),
all in float32 with torch's CPU kernels.

Pinning: ``tests/test_oracle_misc.py`` (``test_cpu_baseline_matches_float64_oracle``,
``test_cpu_dense_baseline_matches_float64_oracle``) checks both against
``oracle.attention.block_sparse_attention`` (float64) on the lists of
``oracle.selector.topk_block_mask`` for the same pooled scores, and on
every block for the dense path.
"""
from __future__ import annotations

import math

import torch


def pooled_prob(q: torch.Tensor, k: torch.Tensor, bq: int = 128, bk: int = 64) -> torch.Tensor:
    def pool(x, b):
        T = x.shape[-2]
        nb = math.ceil(T / b)
        pad = nb * b - T
        xs = torch.nn.functional.pad(x, (0, 0, 0, pad)).view(*x.shape[:-2], nb, b, x.shape[-1]).sum(-2)
        cnt = torch.full((nb,), float(b))
        cnt[-1] = T - (nb - 1) * b
        return xs / cnt.view(nb, 1)

    pq, pk = pool(q, bq), pool(k, bk)
    return torch.softmax(pq @ pk.transpose(-1, -2) / math.sqrt(q.shape[-1]), dim=-1)


def topk_lists(prob: torch.Tensor, sparse_ratio: float, sink: int) -> list:
    kb = prob.shape[-1]
    t = max(int(kb * (1 - sparse_ratio)), 1)
    idx = torch.topk(prob, t, dim=-1).indices
    sinks = torch.arange(kb, kb + sink).expand(*idx.shape[:-1], sink)
    return torch.sort(torch.cat([idx, sinks], dim=-1), dim=-1).values


def topk_layer(q_patch: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sparse_ratio: float) -> torch.Tensor:
    """``[B,H,Np,D]`` output of one Top-K sparse global-attention op (fp32)."""
    B, H, Np, D = q_patch.shape
    Tk = k.shape[-2]
    prob = pooled_prob(q_patch, k[..., :Np, :])
    sink = math.ceil(Tk / 64) - prob.shape[-1]
    lists = topk_lists(prob, sparse_ratio, sink)
    scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q_patch)
    offs = torch.arange(64)
    for b in range(B):
        for h in range(H):
            for i in range(prob.shape[-2]):
                keys = (lists[b, h, i].view(-1, 1) * 64 + offs).view(-1)
                keys = keys[keys < Tk]
                qs = q_patch[b, h, i * 128:(i + 1) * 128]
                s = (qs @ k[b, h, keys].T) * scale
                out[b, h, i * 128:(i + 1) * 128] = torch.softmax(s, dim=-1) @ v[b, h, keys]
    return out


def dense_layer(q_patch: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rows: int = 2048) -> torch.Tensor:
    """``[B,H,Np,D]`` output of exact softmax attention over every key (fp32),
    ``rows`` query rows at a time so the logits stay within a few hundred MB."""
    B, H, Np, D = q_patch.shape
    scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q_patch)
    for b in range(B):
        for h in range(H):
            for r in range(0, Np, rows):
                s = (q_patch[b, h, r:r + rows] @ k[b, h].T) * scale
                out[b, h, r:r + rows] = torch.softmax(s, dim=-1) @ v[b, h]
    return out

