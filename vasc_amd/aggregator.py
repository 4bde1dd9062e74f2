"""VGGT/Pi3-shaped attention modules with random initialisation.

The reference patches the global attention modules of the upstream VGGT
and Pi3 models (``vggt.py:215-299``, ``pi3.py:138-233``); those packages and
their checkpoints are not part of the reference tree, so this module
provides modules of the same shape for the benchmarks and tests:

* ``RotaryPositionEmbedding2D``: the 2D rotary embedding the upstream
  attention applies as ``rope(q, pos)`` (``attention.py:8359-8361``):
  features ``[0, D/2)`` rotate with a token's row position, ``[D/2, D)``
  with its column position, with frequencies ``base**(-2j/(D/2))``. The
  cos/sin tables are computed once on the host and shared by the torch
  path and the fused layout kernel.
* ``Attention``: ``qkv`` (Linear dim -> 3 dim), per-head ``q_norm`` /
  ``k_norm`` (LayerNorm), ``rope``, ``proj`` and ``proj_drop``, the fields
  ``adaptive_sparse_attention_forward`` reads. Its own ``forward`` is the
  dense layer on this build's MFMA attention kernel.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import ops


class RotaryPositionEmbedding2D(nn.Module):
    """2D rotary position embedding with host-computed cos/sin tables."""

    def __init__(self, frequency: float = 100.0):
        super().__init__()
        self.base_frequency = float(frequency)
        self._tables: dict = {}

    def tables(self, n_positions: int, head_dim: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        """float32 ``(cos, sin)`` of ``p * base**(-2j/(head_dim/2))``, shape ``[n, head_dim/4]``."""
        n = max(int(n_positions), 1)
        key = (head_dim, str(device))
        have = self._tables.get(key)
        if have is None or have[0].shape[0] < n:
            half = head_dim // 2
            inv = 1.0 / (self.base_frequency ** (torch.arange(0, half, 2, dtype=torch.float64) / half))
            ang = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
            have = (ang.cos().float().to(device), ang.sin().float().to(device))
            self._tables[key] = have
        return have

    def forward(self, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """tokens ``[B,H,T,D]``, positions ``[B,T,2]`` integer (row, column)."""
        D = tokens.shape[-1]
        q4 = D // 4
        cos, sin = self.tables(int(positions.max()) + 1, D, tokens.device)
        x = tokens.float()
        out = torch.empty_like(x)
        for half in range(2):
            p = positions[..., half].long()
            c, s = cos[p][:, None], sin[p][:, None]  # [B,1,T,D/4]
            lo = x[..., half * 2 * q4: half * 2 * q4 + q4]
            hi = x[..., half * 2 * q4 + q4: (half + 1) * 2 * q4]
            out[..., half * 2 * q4: half * 2 * q4 + q4] = lo * c - hi * s
            out[..., half * 2 * q4 + q4: (half + 1) * 2 * q4] = hi * c + lo * s
        return out.to(tokens.dtype)


class Attention(nn.Module):
    """Multi-head attention of the VGGT/Pi3 blocks (qk-norm, 2D RoPE)."""

    def __init__(self, dim: int = 1024, num_heads: int = 16, qkv_bias: bool = True, qk_norm: bool = True,
                 rope: RotaryPositionEmbedding2D | None = None, norm_eps: float = 1e-6):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.qkv = nn.Linear(dim, 3 * dim, bias=qkv_bias)
        self.q_norm = nn.LayerNorm(self.head_dim, eps=norm_eps) if qk_norm else nn.Identity()
        self.k_norm = nn.LayerNorm(self.head_dim, eps=norm_eps) if qk_norm else nn.Identity()
        self.rope = rope
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Identity()

    def forward(self, x: torch.Tensor, pos: torch.Tensor | None = None) -> torch.Tensor:
        """Dense attention over all tokens of ``x [B,T,dim]`` (one sequence per batch entry)."""
        B, T, dim = x.shape
        H, D = self.num_heads, self.head_dim
        qkv = self.qkv(x).to(torch.bfloat16).view(B, T, 3, H, D)
        qp, _, k, v = ops.pack_qkv(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], 1, T, 0,
                                   q_norm=layer_norm_args(self.q_norm), k_norm=layer_norm_args(self.k_norm),
                                   pos=pos if self.rope is not None else None,
                                   rope_tables=self._tables(pos, D, x.device))
        o = ops.dense_attn(qp, k, ops.pack_v(v), scale=1.0 / math.sqrt(D))
        out = ops.restore_tokens(o, None, 1, T, 0)
        return self.proj_drop(self.proj(out.to(x.dtype)))

    def _tables(self, pos, head_dim, device):
        if self.rope is None or pos is None:
            return None
        return self.rope.tables(int(pos.max()) + 1, head_dim, device)


def layer_norm_args(norm: nn.Module):
    """``(weight, bias, eps)`` of a LayerNorm over the head dimension, None
    for Identity; raises for any other module (the caller then runs it in
    torch)."""
    if isinstance(norm, nn.Identity) or norm is None:
        return None
    if isinstance(norm, nn.LayerNorm) and len(norm.normalized_shape) == 1:
        return (norm.weight, norm.bias, norm.eps)
    raise TypeError(f"{type(norm).__name__} is not a per-head LayerNorm")


def fused_layout_supported(attn: nn.Module) -> bool:
    """Whether the layout kernel can apply this module's q/k norms and rope."""
    try:
        layer_norm_args(getattr(attn, "q_norm", None))
        layer_norm_args(getattr(attn, "k_norm", None))
    except TypeError:
        return False
    rope = getattr(attn, "rope", None)
    return rope is None or isinstance(rope, RotaryPositionEmbedding2D)
