"""CPU restatement of the global layer's token layout, q/k norm and 2D rotary embedding.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

Token layout (reference ``src/sparse_vggt/utils/tokens.py``): frame-major
tokens ``[..., N*P, C]`` hold, per frame, S special tokens then P-S patch
tokens; the global layer works on ``[all patch tokens; all special tokens]``.

* ``get_patch_tokens`` (tokens.py:2-24), ``get_special_tokens`` (27-46),
  ``reorder_to_patch_then_special`` (49-62), ``restore_to_frame_major``
  (102-126).
* ``pack_layer`` follows the layer's order of operations
  (attention.py:8351-8361 then 8419-8469): head split of the qkv
  projection, ``q_norm`` / ``k_norm``, rotary embedding, reorder.
* ``layer_norm`` is torch's ``LayerNorm`` over the last axis (biased
  variance, ``(x - mean) / sqrt(var + eps) * w + b``).
* ``rope_2d`` is the 2D rotary embedding the upstream VGGT/Pi3 attention
  modules apply (their ``rope(q, pos)``; the upstream packages are not part
  of the reference tree): features ``[0, D/2)`` rotate with the row
  position, ``[D/2, D)`` with the column position, and inside a half feature
  ``j < D/4`` pairs with ``j + D/4`` through the angle ``position * freq_j``
  (``x*cos + rotate_half(x)*sin``). The angles enter as cos/sin tables, so
  the restatement and the kernel share them.

Pinning (``tests/test_oracle_layout.py``): the layout functions by explicit
index construction on small inputs, the reorder/restore round trip and the
S = 0 case; ``layer_norm`` against ``torch.nn.functional.layer_norm``;
``rope_2d`` by the closed forms of a rotation (position 0 is the identity,
each feature pair keeps its norm, rotating by p1 then p2 equals rotating by
p1 + p2 for table angles that add) and by a planted sign error that the
checks catch.
"""
from __future__ import annotations

import numpy as np


def _frames(x: np.ndarray, N: int, P: int) -> np.ndarray:
    assert x.shape[-2] == N * P, f"expected {N}*{P} tokens, got {x.shape[-2]}"
    return x.reshape(x.shape[:-2] + (N, P, x.shape[-1]))


def get_patch_tokens(x, N: int, P: int, S: int) -> np.ndarray:
    """tokens.py:2-24: patch tokens ``[..., N*(P-S), C]`` in frame order."""
    f = _frames(np.asarray(x), N, P)
    return f[..., S:, :].reshape(x.shape[:-2] + (N * (P - S), x.shape[-1])).copy()


def get_special_tokens(x, N: int, P: int, S: int):
    """tokens.py:27-46: special tokens ``[..., N*S, C]``, or None when S == 0."""
    if S == 0:
        return None
    f = _frames(np.asarray(x), N, P)
    return f[..., :S, :].reshape(x.shape[:-2] + (N * S, x.shape[-1])).copy()


def reorder_to_patch_then_special(x, N: int, P: int, S: int) -> np.ndarray:
    """tokens.py:49-62: ``[all patch; all special]``."""
    patch = get_patch_tokens(x, N, P, S)
    special = get_special_tokens(x, N, P, S)
    return patch if special is None else np.concatenate([patch, special], axis=-2)


def restore_to_frame_major(x, N: int, P: int, S: int) -> np.ndarray:
    """tokens.py:102-126: inverse of ``reorder_to_patch_then_special``."""
    x = np.asarray(x)
    assert x.shape[-2] == N * P
    n_patch = N * (P - S)
    patch = x[..., :n_patch, :].reshape(x.shape[:-2] + (N, P - S, x.shape[-1]))
    if S:
        special = x[..., n_patch:, :].reshape(x.shape[:-2] + (N, S, x.shape[-1]))
        patch = np.concatenate([special, patch], axis=-2)
    return patch.reshape(x.shape[:-2] + (N * P, x.shape[-1]))


def layer_norm(x, weight=None, bias=None, eps: float = 1e-6) -> np.ndarray:
    """LayerNorm over the last axis in float64."""
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def rope_tables(n_positions: int, head_dim: int, base: float = 100.0):
    """float32 cos/sin tables ``[n_positions, head_dim/4]`` of ``p * base**(-2j/(head_dim/2))``."""
    half = head_dim // 2
    inv_freq = 1.0 / (base ** (np.arange(0, half, 2, dtype=np.float64) / half))
    ang = np.arange(n_positions, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_2d(x, pos, cos, sin) -> np.ndarray:
    """2D rotary embedding of ``x [..., T, D]`` at integer positions ``pos [T, 2]``.

    Uses the tables as given (float32 values, float64 arithmetic).
    """
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    q4 = D // 4
    cos = np.asarray(cos, np.float64)
    sin = np.asarray(sin, np.float64)
    pos = np.asarray(pos, np.int64)
    out = np.empty_like(x)
    for half in range(2):
        p = np.clip(pos[:, half], 0, cos.shape[0] - 1)
        c, s = cos[p], sin[p]                      # [T, D/4]
        lo = x[..., half * 2 * q4: half * 2 * q4 + q4]
        hi = x[..., half * 2 * q4 + q4: (half + 1) * 2 * q4]
        out[..., half * 2 * q4: half * 2 * q4 + q4] = lo * c - hi * s
        out[..., half * 2 * q4 + q4: (half + 1) * 2 * q4] = hi * c + lo * s
    return out


def pack_layer(qkv, N: int, P: int, S: int, H: int, *, q_norm=None, k_norm=None, pos=None, tables=None):
    """qkv projection ``[B, T, 3*H*D]`` -> (q_patch, q_special, k, v) in float64.

    ``q_norm`` / ``k_norm``: ``(weight, bias, eps)`` or None; ``pos [T, 2]``
    with ``tables = (cos, sin)`` applies the rotary embedding.
    """
    qkv = np.asarray(qkv, np.float64)
    B, T, C3 = qkv.shape
    D = C3 // (3 * H)
    x = qkv.reshape(B, T, 3, H, D).transpose(2, 0, 3, 1, 4)  # [3, B, H, T, D]
    q, k, v = x[0], x[1], x[2]
    if q_norm is not None:
        q = layer_norm(q, *q_norm)
    if k_norm is not None:
        k = layer_norm(k, *k_norm)
    if pos is not None:
        q = rope_2d(q, pos, *tables)
        k = rope_2d(k, pos, *tables)
    return (get_patch_tokens(q, N, P, S), get_special_tokens(q, N, P, S),
            reorder_to_patch_then_special(k, N, P, S), reorder_to_patch_then_special(v, N, P, S))
