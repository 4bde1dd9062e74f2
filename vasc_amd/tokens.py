"""Token layout helpers of the global-attention layer (torch, device agnostic).

Same contract as the reference's ``src/sparse_vggt/utils/tokens.py:2-126``:
frame-major tokens ``[..., N*P, C]`` (per frame: S special tokens, then
P-S patch tokens) versus the global layout ``[all patch; all special]``.
"""
from __future__ import annotations

import torch


def _frames(x: torch.Tensor, N: int, P: int) -> torch.Tensor:
    assert x.shape[-2] == N * P, f"expected {N}*{P} tokens, got {x.shape[-2]}"
    return x.reshape(*x.shape[:-2], N, P, x.shape[-1])


def get_patch_tokens(x: torch.Tensor, N: int, P: int, S: int) -> torch.Tensor:
    """Patch tokens ``[..., N*(P-S), C]`` in frame order (contiguous copy)."""
    f = _frames(x, N, P)
    return f[..., S:, :].reshape(*x.shape[:-2], N * (P - S), x.shape[-1]).contiguous()


def get_special_tokens(x: torch.Tensor, N: int, P: int, S: int):
    """Special tokens ``[..., N*S, C]``, or None when S == 0."""
    if S == 0:
        return None
    f = _frames(x, N, P)
    return f[..., :S, :].reshape(*x.shape[:-2], N * S, x.shape[-1])


def reorder_to_patch_then_special(x: torch.Tensor, N: int, P: int, S: int) -> torch.Tensor:
    """``[all patch tokens; all special tokens]`` (one contiguous copy)."""
    f = _frames(x, N, P)
    out = torch.empty_like(x)
    n_patch = N * (P - S)
    out[..., :n_patch, :].view(*x.shape[:-2], N, P - S, x.shape[-1]).copy_(f[..., S:, :])
    if S:
        out[..., n_patch:, :].view(*x.shape[:-2], N, S, x.shape[-1]).copy_(f[..., :S, :])
    return out


def restore_to_frame_major(x: torch.Tensor, N: int, P: int, S: int) -> torch.Tensor:
    """Inverse of ``reorder_to_patch_then_special``."""
    assert x.shape[-2] == N * P
    n_patch = N * (P - S)
    out = torch.empty_like(x)
    f = out.view(*x.shape[:-2], N, P, x.shape[-1])
    f[..., S:, :].copy_(x[..., :n_patch, :].reshape(*x.shape[:-2], N, P - S, x.shape[-1]))
    if S:
        f[..., :S, :].copy_(x[..., n_patch:, :].reshape(*x.shape[:-2], N, S, x.shape[-1]))
    return out
