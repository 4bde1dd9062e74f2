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
* ``Block`` (pre-norm attention + MLP with LayerScale), ``Aggregator``
  (VGGT: 24 frame / 24 global blocks, 1 camera + 4 register tokens per
  frame, readouts at layers 4, 11, 17, 23; vggt.py:64-212) and
  ``Pi3Decoder`` (36 blocks, odd ones global, 5 register tokens;
  pi3.py:70-135). The upstream DINOv2 patch embedding is replaced by one
  14x14 convolution. ``vasc_amd.install`` patches their global blocks.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import ops
from .attention import frame_grid


class RotaryPositionEmbedding2D(nn.Module):
    """2D rotary position embedding with host-computed cos/sin tables.

    The tables cover positions ``[0, MAX_POSITIONS)`` (a grid of up to 4096
    patches per side); larger positions are clamped to the last entry, by
    the layout kernel and by ``forward`` alike, so no call has to read the
    positions back to size the tables.
    """

    MAX_POSITIONS = 4096

    def __init__(self, frequency: float = 100.0):
        super().__init__()
        self.base_frequency = float(frequency)
        self._tables: dict = {}

    def tables(self, head_dim: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        """float32 ``(cos, sin)`` of ``p * base**(-2j/(head_dim/2))``, shape ``[MAX_POSITIONS, head_dim/4]``."""
        key = (head_dim, str(device))
        have = self._tables.get(key)
        if have is None:
            half = head_dim // 2
            inv = 1.0 / (self.base_frequency ** (torch.arange(0, half, 2, dtype=torch.float64) / half))
            ang = torch.arange(self.MAX_POSITIONS, dtype=torch.float64)[:, None] * inv[None, :]
            have = (ang.cos().float().to(device), ang.sin().float().to(device))
            self._tables[key] = have
        return have

    def forward(self, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """tokens ``[B,H,T,D]``, positions ``[B,T,2]`` integer (row, column)."""
        D = tokens.shape[-1]
        q4 = D // 4
        cos, sin = self.tables(D, tokens.device)
        x = tokens.float()
        out = torch.empty_like(x)
        for half in range(2):
            p = positions[..., half].long().clamp(0, self.MAX_POSITIONS - 1)
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
        qp, _, k, _ = ops.pack_qkv(qkv[:, :, 0], qkv[:, :, 1], None, 1, T, 0,
                                   q_norm=layer_norm_args(self.q_norm), k_norm=layer_norm_args(self.k_norm),
                                   pos=pos if self.rope is not None else None,
                                   rope_tables=self._tables(pos, D, x.device))
        # V needs neither norm nor rotation: its MFMA tiles are packed straight
        # from the projection's strided rows
        vt = ops.pack_v(qkv[:, :, 2].transpose(1, 2))
        # the kernel writes straight into the frame-major [B, T, H*D] rows proj reads
        out = torch.empty(B, T, H * D, device=x.device, dtype=torch.bfloat16)
        ops.dense_attn(qp, k, vt, scale=1.0 / math.sqrt(D), out=out.view(B, T, H, D).transpose(1, 2))
        return self.proj_drop(self.proj(out.to(x.dtype)))

    def _tables(self, pos, head_dim, device):
        if self.rope is None or pos is None:
            return None
        return self.rope.tables(head_dim, device)


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


class Mlp(nn.Module):
    def __init__(self, dim: int, hidden: int):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


class LayerScale(nn.Module):
    def __init__(self, dim: int, init_values: float = 0.01):
        super().__init__()
        self.gamma = nn.Parameter(torch.full((dim,), float(init_values)))

    def forward(self, x):
        return x * self.gamma


class Block(nn.Module):
    """Pre-norm transformer block: ``x + ls1(attn(norm1(x))) + ls2(mlp(norm2(.)))``."""

    def __init__(self, dim: int = 1024, num_heads: int = 16, mlp_ratio: float = 4.0,
                 rope: RotaryPositionEmbedding2D | None = None, init_values: float = 0.01):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim, eps=1e-6)
        self.attn = Attention(dim, num_heads, rope=rope)
        self.ls1 = LayerScale(dim, init_values)
        self.norm2 = nn.LayerNorm(dim, eps=1e-6)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.ls2 = LayerScale(dim, init_values)

    def forward(self, x: torch.Tensor, pos: torch.Tensor | None = None, *, normed: torch.Tensor | None = None,
                next_norm: nn.LayerNorm | None = None):
        """``normed``: ``norm1(x)`` when the caller already has it; with
        ``next_norm`` also returns ``next_norm`` of the output (the next
        block's first norm), as ``(out, normed_out)``. On the GPU in bf16
        each residual update runs with the norm after it as one
        ``vasc_residual_norm`` pass, rounded as the separate torch ops."""
        h = self.norm1(x) if normed is None else normed
        a = self.attn(h, pos=pos)
        if not _fused_residual(x, a, self, next_norm):
            x = x + self.ls1(a)
            x = x + self.ls2(self.mlp(self.norm2(x)))
            return x if next_norm is None else (x, next_norm(x))
        x, h2 = ops.residual_norm(x, a, self.ls1.gamma, _ln(self.norm2))
        x, nxt = ops.residual_norm(x, self.mlp(h2), self.ls2.gamma, _ln(next_norm) if next_norm is not None else None)
        return x if next_norm is None else (x, nxt)


def _fused_residual(x: torch.Tensor, y: torch.Tensor, blk: "Block", next_norm: nn.LayerNorm | None) -> bool:
    """The fused pass rounds as torch's bf16 ops do on bf16 activations and
    bf16 parameters; anything else (fp32 parameters under autocast, where
    torch promotes the products and the LayerNorm to fp32) takes the torch ops."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16 and x.shape == y.shape
            and x.shape[-1] in (512, 1024, 1536, 2048)):
        return False
    params = [blk.ls1.gamma, blk.ls2.gamma, blk.norm2.weight, blk.norm2.bias]
    if next_norm is not None:
        params += [next_norm.weight, next_norm.bias]
    return all(p is None or p.dtype == torch.bfloat16 for p in params)


def _ln(norm: nn.LayerNorm):
    return (norm.weight, norm.bias, norm.eps)


def patch_tokens(conv: nn.Conv2d, x: torch.Tensor) -> torch.Tensor:
    """``conv(x).flatten(2).transpose(1, 2)`` for the patch embedding: a
    convolution whose stride equals its kernel (no padding, dilation or
    groups) is one GEMM over the non-overlapping patches, which hipBLASLt
    runs far faster than the library's im2col path for a 3-channel input."""
    p = conv.kernel_size
    if not (conv.stride == p and conv.padding == (0, 0) and conv.dilation == (1, 1) and conv.groups == 1):
        return conv(x).flatten(2).transpose(1, 2)
    BN, C, Hi, Wi = x.shape
    h, w = Hi // p[0], Wi // p[1]
    x = x[:, :, :h * p[0], :w * p[1]]
    patches = x.reshape(BN, C, h, p[0], w, p[1]).permute(0, 2, 4, 1, 3, 5).reshape(BN * h * w, C * p[0] * p[1])
    out = nn.functional.linear(patches, conv.weight.reshape(conv.out_channels, -1), conv.bias)
    return out.view(BN, h * w, conv.out_channels)


def grid_positions(frames: int, h: int, w: int, special: int, device) -> torch.Tensor:
    """``[frames, special + h*w, 2]`` integer (row, column) positions: patch
    tokens get ``(y+1, x+1)``, special tokens ``(0, 0)`` (vggt.py:122-131)."""
    ys, xs = torch.meshgrid(torch.arange(h, device=device), torch.arange(w, device=device), indexing="ij")
    patch = torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1
    pos = torch.cat([torch.zeros(special, 2, dtype=patch.dtype, device=device), patch])
    return pos.unsqueeze(0).expand(frames, -1, -1)


class Aggregator(nn.Module):
    """VGGT-shaped alternating frame/global attention aggregator.

    The upstream patch embedding is a DINOv2 ViT; here it is one 14x14
    convolution (the benchmark measures the attention blocks). Tokens per
    frame: 1 camera + ``num_register_tokens`` registers + the patches; the
    first frame uses its own camera/register tokens (slice_expand_and_flatten).
    Frame blocks attend inside each frame, global blocks across all frames.
    """

    def __init__(self, dim: int = 1024, depth: int = 24, num_heads: int = 16, mlp_ratio: float = 4.0,
                 patch_size: int = 14, num_register_tokens: int = 4, camera_token: bool = True,
                 intermediate_layer_idx=(4, 11, 17, 23)):
        super().__init__()
        self.patch_size = patch_size
        self.patch_embed = nn.Conv2d(3, dim, patch_size, patch_size)
        self.rope = RotaryPositionEmbedding2D(100.0)
        self.frame_blocks = nn.ModuleList([Block(dim, num_heads, mlp_ratio, self.rope) for _ in range(depth)])
        self.global_blocks = nn.ModuleList([Block(dim, num_heads, mlp_ratio, self.rope) for _ in range(depth)])
        self.camera_token = nn.Parameter(torch.randn(1, 2, 1, dim) * 1e-6) if camera_token else None
        self.register_token = nn.Parameter(torch.randn(1, 2, num_register_tokens, dim) * 1e-6)
        self.patch_start_idx = int(camera_token) + num_register_tokens
        self.aa_block_num = depth
        self.intermediate_layer_idx = list(intermediate_layer_idx)
        self.register_buffer("_resnet_mean", torch.tensor([0.485, 0.456, 0.406]).view(1, 1, 3, 1, 1), persistent=False)
        self.register_buffer("_resnet_std", torch.tensor([0.229, 0.224, 0.225]).view(1, 1, 3, 1, 1), persistent=False)

    @staticmethod
    def _expand(token: torch.Tensor, B: int, N: int) -> torch.Tensor:
        first = token[:, :1].expand(B, 1, *token.shape[2:])
        rest = token[:, 1:].expand(B, N - 1, *token.shape[2:])
        return torch.cat([first, rest], dim=1).reshape(B * N, *token.shape[2:])

    def forward(self, images: torch.Tensor):
        """images ``[B, N, 3, H, W]`` in [0, 1] -> (list of per-layer outputs, patch_start_idx)."""
        routing_state = getattr(self, "_sparse_routing_state", None)
        if routing_state is not None:
            routing_state.clear()
        B, N, _, Hi, Wi = images.shape
        x = ((images - self._resnet_mean) / self._resnet_std).view(B * N, 3, Hi, Wi).to(self.patch_embed.weight.dtype)
        tokens = patch_tokens(self.patch_embed, x)
        special = [self._expand(self.register_token, B, N)]
        if self.camera_token is not None:
            special.insert(0, self._expand(self.camera_token, B, N))
        tokens = torch.cat([*(s.to(tokens.dtype) for s in special), tokens], dim=1)
        h, w = Hi // self.patch_size, Wi // self.patch_size
        P, C = tokens.shape[1], tokens.shape[2]
        # int32 positions made once: the layers' layout kernel reads them as they are
        pos = grid_positions(B * N, h, w, self.patch_start_idx, images.device).to(torch.int32).contiguous()
        pos_global = pos.view(B, N * P, 2)
        outputs = []
        normed = None  # the next block's norm1 of the tokens, from the previous block's last pass
        with frame_grid(h, w):
            for i in range(self.aa_block_num):
                fb, gb = self.frame_blocks[i], self.global_blocks[i]
                tokens, normed = fb(tokens.view(B * N, P, C), pos=pos, normed=normed, next_norm=gb.norm1)
                frame_out = tokens.view(B, N, P, C)
                nxt = self.frame_blocks[i + 1].norm1 if i + 1 < self.aa_block_num else None
                out = gb(tokens.view(B, N * P, C), pos=pos_global, normed=normed.view(B, N * P, C), next_norm=nxt)
                tokens, normed = out if nxt is not None else (out, None)
                if normed is not None:
                    normed = normed.view(B * N, P, C)
                if i in self.intermediate_layer_idx:
                    outputs.append(torch.cat([frame_out, tokens.view(B, N, P, C)], dim=-1))
                else:
                    outputs.append(None)
        _finalize(self)
        return outputs, self.patch_start_idx


class Pi3Decoder(nn.Module):
    """Pi3-shaped decoder: alternating frame (even) / global (odd) blocks over
    5 register tokens + the patch tokens of each frame (pi3.py:70-135)."""

    def __init__(self, dim: int = 1024, depth: int = 36, num_heads: int = 16, mlp_ratio: float = 4.0,
                 patch_size: int = 14, num_register_tokens: int = 5):
        super().__init__()
        self.patch_size = patch_size
        self.patch_embed = nn.Conv2d(3, dim, patch_size, patch_size)
        self.rope = RotaryPositionEmbedding2D(100.0)
        self.decoder = nn.ModuleList([Block(dim, num_heads, mlp_ratio, self.rope) for _ in range(depth)])
        self.register_token = nn.Parameter(torch.randn(1, 1, num_register_tokens, dim) * 1e-6)
        self.patch_start_idx = num_register_tokens

    def forward(self, images: torch.Tensor):
        """images ``[B, N, 3, H, W]`` -> (concatenated last two outputs, positions)."""
        B, N, _, Hi, Wi = images.shape
        x = images.view(B * N, 3, Hi, Wi).to(self.patch_embed.weight.dtype)
        hidden = patch_tokens(self.patch_embed, x)
        return self.decode(hidden, N, Hi, Wi)

    def decode(self, hidden: torch.Tensor, N: int, H: int, W: int):
        routing_state = getattr(self, "_sparse_routing_state", None)
        if routing_state is not None:
            routing_state.clear()
        BN, hw, C = hidden.shape
        B = BN // N
        reg = self.register_token.repeat(B, N, 1, 1).reshape(B * N, *self.register_token.shape[-2:])
        hidden = torch.cat([reg.to(hidden.dtype), hidden], dim=1)
        hw = hidden.shape[1]
        h, w = H // self.patch_size, W // self.patch_size
        pos = grid_positions(B * N, h, w, self.patch_start_idx, hidden.device).to(torch.int32).contiguous()
        pos_frame, pos_global = pos.view(B * N, hw, 2), pos.view(B, N * hw, 2)
        final = []
        normed = None  # the next block's norm1, from the previous block's last pass
        depth = len(self.decoder)
        with frame_grid(h, w):
            for i, blk in enumerate(self.decoder):
                shape = (B * N, hw, C) if i % 2 == 0 else (B, N * hw, C)
                nxt = self.decoder[i + 1].norm1 if i + 1 < depth else None
                out = blk(hidden.reshape(shape), pos=pos_frame if i % 2 == 0 else pos_global,
                          normed=normed.view(shape) if normed is not None else None, next_norm=nxt)
                hidden, normed = out if nxt is not None else (out, None)
                if i + 1 in (depth - 1, depth):
                    final.append(hidden.reshape(B * N, hw, C))
        _finalize(self)
        return torch.cat(final, dim=-1), pos


def _finalize(model: nn.Module) -> None:
    """Terminal ledger settlement after the last layer (vggt.py:193-204, pi3.py:23-36)."""
    routing_state = getattr(model, "_sparse_routing_state", None)
    if routing_state is None:
        return
    from .sparse_wrapper import finalize_cosa_value_risk_pair_debt
    store = getattr(model, "_sparse_aux_output_store", None)
    stats = None
    if store:
        last = store[max(store)]
        stats = last if isinstance(last, dict) else None
    finalize_cosa_value_risk_pair_debt(routing_state, stats_store=stats)
