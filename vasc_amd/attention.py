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

import contextlib
import contextvars
import math

import torch

from . import ops


def predict_attention(query: torch.Tensor, key: torch.Tensor, ks_q: int = 128, ks_k: int = 64,
                      pool_mode: str = "avg", return_key_block_variance: bool = False) -> torch.Tensor:
    """Pooled attention probabilities ``[B,H,ceil(Tq/ks_q),ceil(Tk/ks_k)]`` (fp32).

    Pooled means are rounded to bf16 (block maxima are exact) and the logits
    follow the bf16 matmul of the reference's autocast run; the softmax is
    fp32. With ``return_key_block_variance`` also the per-key-block variance
    proxy ``[B,H,Kb]`` (ATT:69-89): the block mean of the squared token norms
    (squares rounded to the key dtype, float32 sums) minus the squared norm
    of the bf16 block mean, clamped at 0.
    """
    assert pool_mode in ("max", "avg"), f"{pool_mode=}"
    assert query.ndim == 4 and key.ndim == 4
    if (ks_q, ks_k) != (ops.BLOCK_Q, ops.BLOCK_K):
        raise NotImplementedError("pooling is built for 128-token query and 64-token key blocks")
    if pool_mode == "max":
        pq, pk = ops.pool_qk_max(query, key)
    else:
        pq, pk, _, _ = ops.pool_qkv(q=query, k=key, innovation=False)
    prob = ops.pooled_softmax(pq, pk, scale=1.0 / math.sqrt(query.shape[-1]))
    if not return_key_block_variance:
        return prob
    mean = pk if pool_mode == "avg" else ops.pool_qkv(k=key, innovation=False)[1]
    tok = (key * key).sum(dim=-1, dtype=torch.float32)  # squares in the key dtype, float32 sums: [B,H,Tk]
    Tk = tok.shape[-1]
    nb = mean.shape[-2]
    padded = torch.nn.functional.pad(tok, (0, nb * ops.BLOCK_K - Tk))
    count = torch.full((nb,), float(ops.BLOCK_K), device=tok.device)
    count[-1] = Tk - (nb - 1) * ops.BLOCK_K
    mean_sq = padded.view(*tok.shape[:-1], nb, ops.BLOCK_K).sum(-1) / count
    var = (mean_sq - mean.float().square().sum(dim=-1)).clamp_min(0.0)
    return prob, var


_FRAME_GRID: contextvars.ContextVar = contextvars.ContextVar("vasc_frame_grid", default=None)


@contextlib.contextmanager
def frame_grid(h: int, w: int):
    """Announce the patch grid of the frames for the layers run inside.

    The layer forward otherwise reads the grid back from the positions
    (ATT:8343-8349), a device-to-host copy in every layer; model forwards
    that built the positions themselves pass the grid here instead.
    """
    token = _FRAME_GRID.set((int(h), int(w)))
    try:
        yield
    finally:
        _FRAME_GRID.reset(token)


def _infer_frames(pos: torch.Tensor, n_tokens: int, S: int):
    """H, W, N, P from the RoPE positions (ATT:8343-8349): patch positions are
    1-based (specials sit at 0), so the maxima are the grid sizes."""
    grid = _FRAME_GRID.get()
    if grid is not None:
        H, W = grid
    else:
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

    The head split, q/k norms, rotary embedding and [patch; special] reorder
    (ATT:8351-8469) are one layout kernel when the norms are per-head
    LayerNorms (or identities) and the rope is ``RotaryPositionEmbedding2D``;
    other modules run their norms and rope in torch first. Special-token
    queries attend to every key in the same launch as the patch queries, and
    that launch writes every result on its frame-major token row, the order
    ``proj`` reads (the reference's restore and transpose, ATT:8992-9030).
    With a PV post-cut the separate restore kernel does that step.
    """
    from .aggregator import fused_layout_supported, layer_norm_args
    from .launcher import routing_config
    from .sparse_wrapper import sparse_global_attention

    if routing_state is None:
        routing_state = getattr(self, "_sparse_routing_state", None)
    B, NP, dim = x.shape
    S, nh = num_special_tokens, num_heads
    hd = dim // nh
    Hp, Wp, N, P = _infer_frames(pos, NP, S)
    qkv = self.qkv(x).to(torch.bfloat16).view(B, NP, 3, nh, hd)
    rope = getattr(self, "rope", None)
    n_patch = N * (P - S)
    vasc_mode = routing_config().mode == "vasc"
    if pool_mode == "avg" and n_patch > 0 and fused_layout_supported(self):
        # layout, V tiles, block means and value innovation in one pass
        tables = rope.tables(hd, x.device) if rope is not None else None
        q_patch, q_special, k_re, vt, pq, pk, innovation, _ = ops.pack_global(
            qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S, q_norm=layer_norm_args(self.q_norm),
            k_norm=layer_norm_args(self.k_norm), pos=pos if rope is not None else None, rope_tables=tables,
            innovation=vasc_mode)
        # the ledger's QK-order priority (the cleaned score) from the same launch
        attn_pooled, priority = ops.pooled_softmax(pq, pk, scale=1.0 / math.sqrt(hd), priority=True) \
            if vasc_mode else (ops.pooled_softmax(pq, pk, scale=1.0 / math.sqrt(hd)), None)
        tokens_out, _, sparsity = sparse_global_attention(
            q_patch, q_special, k_re, None, attn_pooled, sparse_ratio=sparse_ratio, cdf_threshold=cdf_threshold,
            layer_idx=layer_idx, routing_state=routing_state, num_patch_tokens=n_patch,
            want_sparsity=aux_output_store is not None, _innovation=innovation, token_layout=(N, P, S), _vt=vt,
            _priority=priority, **research)
        return _finish(self, x, tokens_out, sparsity, aux_output_store)
    if fused_layout_supported(self):
        tables = rope.tables(hd, x.device) if rope is not None else None
        q_patch, q_special, k_re, v_re = ops.pack_qkv(
            qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S, q_norm=layer_norm_args(self.q_norm),
            k_norm=layer_norm_args(self.k_norm), pos=pos if rope is not None else None, rope_tables=tables)
    else:
        q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
        q, k = self.q_norm(q), self.k_norm(k)
        if rope is not None:
            q, k = rope(q, pos), rope(k, pos)
        q_patch, q_special, k_re, v_re = ops.pack_qkv(
            *(t.to(torch.bfloat16).transpose(1, 2) for t in (q, k, v)), N, P, S)
    innovation = None
    if pool_mode == "avg" and vasc_mode:
        # Q, K and V pooled in one pass: predict_attention's pooled Q/K and
        # the selector's value innovation
        pq, pk, _, innovation = ops.pool_qkv(q_patch, k_re[:, :, :n_patch], v_re[:, :, :n_patch])
        attn_pooled = ops.pooled_softmax(pq, pk, scale=1.0 / math.sqrt(hd))
    else:
        attn_pooled = predict_attention(q_patch, k_re[:, :, :n_patch], pool_mode=pool_mode)
    tokens_out, _, sparsity = sparse_global_attention(
        q_patch, q_special, k_re, v_re, attn_pooled, sparse_ratio=sparse_ratio, cdf_threshold=cdf_threshold,
        layer_idx=layer_idx, routing_state=routing_state, num_patch_tokens=n_patch,
        want_sparsity=aux_output_store is not None, _innovation=innovation, token_layout=(N, P, S), **research)
    return _finish(self, x, tokens_out, sparsity, aux_output_store)


def _finish(self, x: torch.Tensor, tokens_out: torch.Tensor, sparsity, aux_output_store: dict | None):
    """Output projection of the frame-major attention output (ATT:9028-9031)."""
    if aux_output_store is not None:
        aux_output_store["sparsity"] = sparsity
    out = self.proj(tokens_out.to(x.dtype))  # already in frame-major token order
    drop = getattr(self, "proj_drop", None)
    return drop(out) if drop is not None else out
