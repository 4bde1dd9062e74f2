"""Pooled predictor and the sparse global-attention layer forward.

Mirrors ``src/sparse_vggt/models/attention.py`` (``ATT``) of the reference:

* ``predict_attention`` (ATT:31-104): block mean pooling of Q (128 tokens)
  and K (64 tokens) and the pooled softmax, on kernels 1a/1b.
* ``adaptive_sparse_attention_forward`` (ATT:8157-9031, release branch):
  qkv, q/k norm, RoPE, reorder to ``[patch; special]``, special-token
  queries attend densely to all keys, patch queries go through
  ``block_sparse_attn_cuda``, restore to frame-major order, projection.
"""
from __future__ import annotations

import math

import torch

from . import ops
from .sparse_wrapper import block_sparse_attn_cuda
from .tokens import get_patch_tokens, get_special_tokens, reorder_to_patch_then_special, restore_to_frame_major


def predict_attention(query: torch.Tensor, key: torch.Tensor, ks_q: int = 128, ks_k: int = 64,
                      pool_mode: str = "avg", return_key_block_variance: bool = False) -> torch.Tensor:
    """Pooled attention probabilities ``[B,H,ceil(Tq/ks_q),ceil(Tk/ks_k)]`` (fp32).

    Pooled means are rounded to bf16 and the logits follow the bf16 matmul
    of the reference's autocast run; the softmax is fp32.
    """
    assert pool_mode in ("max", "avg"), f"{pool_mode=}"
    assert query.ndim == 4 and key.ndim == 4
    if pool_mode != "avg":
        raise NotImplementedError("max pooling is not built (the release modes pool with avg)")
    if (ks_q, ks_k) != (ops.BLOCK_Q, ops.BLOCK_K):
        raise NotImplementedError("pooling is built for 128-token query and 64-token key blocks")
    if return_key_block_variance:
        raise NotImplementedError("key block variance feeds a research router that is not built")
    pq, pk, _, _ = ops.pool_qkv(q=query, k=key, innovation=False)
    return ops.pooled_softmax(pq, pk, scale=1.0 / math.sqrt(query.shape[-1]))


def _infer_frames(pos: torch.Tensor, n_tokens: int, S: int):
    """H, W, N, P from the RoPE positions (ATT:8343-8349): patch positions are
    1-based (specials sit at 0), so the maxima are the grid sizes."""
    H = int(pos[0].max(0).values[0])
    W = int(pos[0].max(0).values[1])
    P = H * W + S
    N = n_tokens // P
    assert N * P == n_tokens, f"{N=}, {H=}, {W=}, {S=}, {n_tokens=}"
    return H, W, N, P


def adaptive_sparse_attention_forward(self, x: torch.Tensor, pos: torch.Tensor, sparse_ratio: float | None = None,
                                      cdf_threshold: float | None = None, pool_mode: str = "avg",
                                      aux_sparsity_only: bool = True, aux_output_store: dict | None = None,
                                      num_special_tokens: int = 5, num_heads: int = 16, *, layer_idx: int = 0,
                                      routing_state: dict | None = None, **research) -> torch.Tensor:
    """Global attention of one layer with the sparse operator (ATT:8157-9031).

    ``self`` provides ``qkv``, ``q_norm``, ``k_norm``, optional ``rope`` and
    ``proj`` / ``proj_drop`` (the upstream VGGT/Pi3 attention module).
    """
    if routing_state is None:
        routing_state = getattr(self, "_sparse_routing_state", None)
    B, NP, dim = x.shape
    S, nh = num_special_tokens, num_heads
    hd = dim // nh
    Hp, Wp, N, P = _infer_frames(pos, NP, S)
    qkv = self.qkv(x).reshape(B, NP, 3, nh, hd).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    q, k = self.q_norm(q), self.k_norm(k)
    if getattr(self, "rope", None) is not None:
        q = self.rope(q, pos)
        k = self.rope(k, pos)
    k_re = reorder_to_patch_then_special(k, N, P, S)
    v_re = reorder_to_patch_then_special(v, N, P, S)
    q_patch = get_patch_tokens(q, N, P, S)
    q_special = get_special_tokens(q, N, P, S)
    n_patch = N * (P - S)
    scale = 1.0 / math.sqrt(hd)
    x_special = None
    if q_special is not None:
        # every special query attends to all tokens: the dense MFMA kernel
        x_special = ops.dense_attn(q_special, k_re, ops.pack_v(v_re), scale=scale).to(q.dtype)
    attn_pooled = predict_attention(q_patch, k_re[:, :, :n_patch], pool_mode=pool_mode)
    x_patch, sparsity = block_sparse_attn_cuda(q_patch, k_re, v_re, attn_pooled, sparse_ratio=sparse_ratio,
                                               cdf_threshold=cdf_threshold, return_sparsity=True,
                                               layer_idx=layer_idx, routing_state=routing_state,
                                               num_patch_tokens=n_patch, **research)
    if aux_output_store is not None:
        aux_output_store["sparsity"] = sparsity
    x_re = torch.cat([x_patch.to(q.dtype), x_special], dim=-2) if x_special is not None else x_patch.to(q.dtype)
    out = restore_to_frame_major(x_re, N, P, S)
    out = out.transpose(1, 2).reshape(B, NP, nh * hd)
    out = self.proj(out)
    drop = getattr(self, "proj_drop", None)
    return drop(out) if drop is not None else out
