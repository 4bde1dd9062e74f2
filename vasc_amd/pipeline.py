"""Device-resident sparse global-attention op for one layer (kernels 1-4).

This is the composition behind ``predict_attention`` followed by
``block_sparse_attn_cuda`` (``attention.py:8714-8892`` ->
``sparse_wrapper.py:6868-8245`` of the reference) with the ledger kept as
device tensors instead of a dict of tensors. The drop-in API in
``vasc_amd.sparse_wrapper`` maps the reference's ``routing_state`` onto this.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import _lib, ops

BLOCK_Q = ops.BLOCK_Q
BLOCK_K = ops.BLOCK_K


def ratio_to_topk(key_blocks: int, sparse_ratio: float) -> int:
    """``int(k_blk * (1 - sparse_ratio))`` (sparse_wrapper.py:1226-1228)."""
    return int(key_blocks * (1 - sparse_ratio))


@dataclass
class Ledger:
    """VASC cross-layer memory of one forward pass (per model)."""
    debt: torch.Tensor | None = None
    pending: torch.Tensor | None = None
    service: torch.Tensor | None = None
    pending_layer: int | None = None
    extra: dict = field(default_factory=dict)

    def clear(self) -> None:
        self.debt = self.pending = self.service = None
        self.pending_layer = None
        self.extra.clear()


@dataclass
class LayerPlan:
    """Static block geometry of one global layer."""
    n_patch: int
    n_total: int
    q_blocks: int
    k_blocks: int
    sink: int
    mixed_tail: bool

    @classmethod
    def make(cls, n_patch: int, n_total: int) -> "LayerPlan":
        kb = math.ceil(n_patch / BLOCK_K)
        return cls(n_patch, n_total, math.ceil(n_patch / BLOCK_Q), kb, math.ceil(n_total / BLOCK_K) - kb,
                   n_patch < n_total and n_patch % BLOCK_K != 0)


def select_layer(prob: torch.Tensor, iota: torch.Tensor | None, plan: LayerPlan, *, mode: str,
                 sparse_ratio: float, official_mask: bool, ledger: Ledger | None, layer_idx: int,
                 want_mask: bool = False, want_priority: bool = False, workspace=None) -> dict:
    """Kernel 2 for one layer with the reference's mixed-tail and hint rules."""
    topk = ratio_to_topk(plan.k_blocks, sparse_ratio)
    force_last = plan.mixed_tail and not official_mask
    if mode == "topk":
        return ops.select_blocks(prob, mode=_lib.MODE_TOPK, topk=topk, force_last=force_last,
                                 sink_blocks=plan.sink, want_mask=want_mask)
    if mode != "vasc":
        raise ValueError(f"unknown selection mode {mode!r}")
    hint = topk + int(force_last)
    out = ops.select_blocks(prob, mode=_lib.MODE_VASC, topk=topk, innovation=iota, force_last=force_last,
                            max_capacity=hint, sink_blocks=plan.sink, debt=ledger.debt,
                            pending_arrival=ledger.pending, prev_service=ledger.service,
                            want_mask=want_mask, want_priority=want_priority, workspace=workspace)
    ledger.debt, ledger.pending, ledger.service = out["debt"], out["arrival"], out["service"]
    ledger.pending_layer = int(layer_idx)
    return out


def sparse_attention_layer(q_patch: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, mode: str,
                           sparse_ratio: float, official_mask: bool = True, ledger: Ledger | None = None,
                           layer_idx: int = 0, scale: float | None = None) -> tuple[torch.Tensor, dict]:
    """Kernels 1-4 for one global layer.

    q_patch ``[B,H,Np,D]`` patch queries; k, v ``[B,H,Tk,D]`` in
    ``[patch; special]`` order. Returns ``(o [B,H,Np,D] bf16, selection)``.
    """
    n_patch, n_total = q_patch.shape[2], k.shape[2]
    plan = LayerPlan.make(n_patch, n_total)
    if mode == "dense":
        return ops.dense_attn(q_patch, k, ops.pack_v(v), scale=scale), {}
    want_v = mode == "vasc"
    pq, pk, _, iota = ops.pool_qkv(q_patch, k[:, :, :n_patch], v[:, :, :n_patch] if want_v else None)
    prob = ops.pooled_softmax(pq, pk)
    sel = select_layer(prob, iota, plan, mode=mode, sparse_ratio=sparse_ratio, official_mask=official_mask,
                       ledger=ledger, layer_idx=layer_idx)
    vt = ops.pack_v(v)
    o = ops.block_sparse_attn(q_patch, k, vt, sel["index"], sel["count"], scale=scale)
    sel["prob"] = prob
    return o, sel


def attention_flops(count_index: tuple[torch.Tensor, torch.Tensor], n_q: int, n_k: int, head_dim: int) -> float:
    """Algorithmic flops 4*d*sum(valid q rows x valid keys of listed blocks)."""
    index, count = count_index
    B, H, qb, W = index.shape
    pos = torch.arange(W, device=index.device).view(1, 1, 1, W)
    live = pos < count.unsqueeze(-1)
    blk = index.long().clamp_min(0)
    keys = (n_k - blk * BLOCK_K).clamp(0, BLOCK_K) * live
    rows = (n_q - torch.arange(qb, device=index.device) * BLOCK_Q).clamp(max=BLOCK_Q).view(1, 1, qb)
    return float(4 * head_dim * (keys.sum(-1) * rows).sum().item())
