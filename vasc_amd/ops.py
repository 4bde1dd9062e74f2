"""Torch-facing wrappers of the C-ABI kernels (one per entry point).

Each wrapper validates shapes and dtypes, allocates outputs with torch's
caching allocator, and launches on ``torch.cuda.current_stream()``. Inputs
must be device tensors; nothing here falls back to the CPU.
"""
from __future__ import annotations

import math

import torch

from . import _lib

BLOCK_Q = 128
BLOCK_K = 64
HEAD_DIM = 64


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (the HIP path has no CPU fallback)")


def _bhtd(t: torch.Tensor, name: str) -> torch.Tensor:
    """bf16 [B,H,T,D] with unit stride on D and 16-byte aligned rows."""
    _dev(t, name)
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B,H,T,D], got {tuple(t.shape)}")
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _ptr(t):
    return None if t is None else t.data_ptr()


# ----------------------------------------------------------------- kernel 1
def pool_qkv(q=None, k=None, v=None, *, innovation: bool = True):
    """Block mean pooling (bf16-rounded) of Q (128) and K, V (64) + V pair innovation.

    Returns ``(pooled_q, pooled_k, pooled_v, innovation)`` with ``None`` for
    skipped inputs.
    """
    ref = next(t for t in (q, k, v) if t is not None)
    q = None if q is None else _bhtd(q, "q")
    k = None if k is None else _bhtd(k, "k")
    v = None if v is None else _bhtd(v, "v")
    B, H, _, D = ref.shape
    nq = q.shape[2] if q is not None else 0
    nk = (k if k is not None else v).shape[2] if (k is not None or v is not None) else 0
    dev = ref.device
    pq = torch.empty(B, H, math.ceil(nq / BLOCK_Q), D, device=dev, dtype=torch.bfloat16) if q is not None else None
    pk = torch.empty(B, H, math.ceil(nk / BLOCK_K), D, device=dev, dtype=torch.bfloat16) if k is not None else None
    pv = torch.empty(B, H, math.ceil(nk / BLOCK_K), D, device=dev, dtype=torch.bfloat16) if v is not None else None
    inn = None
    if v is not None and innovation:
        inn = torch.empty(B, H, math.ceil(math.ceil(nk / BLOCK_K) / 2), device=dev, dtype=torch.float32)
    st = lambda t: (0, 0, 0) if t is None else tuple(t.stride()[:3])  # noqa: E731
    _lib.call("vasc_pool_qkv", _ptr(q), *st(q), _ptr(k), *st(k), _ptr(v), *st(v),
              B, H, nq, nk, D, BLOCK_Q, BLOCK_K, _ptr(pq), _ptr(pk), _ptr(pv), _ptr(inn), _stream())
    return pq, pk, pv, inn


def pooled_softmax(pooled_q: torch.Tensor, pooled_k: torch.Tensor, *, scale: float | None = None,
                   round_bf16: bool = True) -> torch.Tensor:
    """fp32 ``softmax(bf16(bf16(pq.pk) * scale))`` over key blocks, ``[B,H,Qb,Kb]``."""
    _dev(pooled_q, "pooled_q")
    _dev(pooled_k, "pooled_k")
    pq = pooled_q.to(torch.bfloat16).contiguous()
    pk = pooled_k.to(torch.bfloat16).contiguous()
    B, H, qb, D = pq.shape
    kb = pk.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    prob = torch.empty(B, H, qb, kb, device=pq.device, dtype=torch.float32)
    ws = torch.empty(_lib.load().vasc_pooled_softmax_workspace_size(B, H, qb, kb), device=pq.device, dtype=torch.uint8)
    _lib.call("vasc_pooled_softmax", pq.data_ptr(), pk.data_ptr(), B, H, qb, kb, D, float(scale),
              int(bool(round_bf16)), prob.data_ptr(), ws.data_ptr(), _stream())
    return prob


def pair_innovation(pooled_value: torch.Tensor) -> torch.Tensor:
    """Pair innovation of float32 pooled values ``[B,H,Kb,D]`` -> ``[B,H,ceil(Kb/2)]``."""
    _dev(pooled_value, "pooled_value")
    pv = pooled_value.float().contiguous()
    B, H, kb, D = pv.shape
    out = torch.empty(B, H, (kb + 1) // 2, device=pv.device, dtype=torch.float32)
    _lib.call("vasc_pair_innovation", pv.data_ptr(), B, H, kb, D, out.data_ptr(), _stream())
    return out


# ----------------------------------------------------------------- kernel 2
def select_workspace(B: int, H: int, Q: int, K: int, device) -> torch.Tensor:
    n = _lib.fn("vasc_select_workspace_size")(B, H, Q, K)
    return torch.empty(max(int(n), 256), device=device, dtype=torch.uint8)


def select_blocks(score: torch.Tensor, *, mode: int, topk: int, innovation=None, row_cap=None,
                  protected_mask=None, force_last: bool = False, max_capacity: int = 0,
                  sink_blocks: int = 0, debt=None, pending_arrival=None, prev_service=None,
                  want_priority: bool = False, want_mask: bool = False, width: int | None = None,
                  workspace: torch.Tensor | None = None):
    """Block selection (kernel 2). Returns a dict of device tensors.

    Keys: ``index`` [B,H,Q,width] int32 ascending, ``count`` [B,H,Q] int32,
    and in VASC mode ``debt``, ``arrival``, ``service`` [B,H,P] float32,
    ``gate`` int32 [1]; optional ``priority`` / ``mask``.
    """
    _dev(score, "score")
    s = score.float().contiguous()
    B, H, Q, K = s.shape
    P = (K + 1) // 2
    vasc = mode == _lib.MODE_VASC
    dev = s.device
    if vasc:
        maxc = min(int(max_capacity), K)
    else:
        maxc = min(max(int(topk), 1) + int(bool(force_last)), K)
    width = maxc + sink_blocks if width is None else int(width)
    out = {
        "index": torch.empty(B, H, Q, max(width, 1), device=dev, dtype=torch.int32),
        "count": torch.empty(B, H, Q, device=dev, dtype=torch.int32),
    }
    f32 = lambda t: None if t is None else t.float().contiguous()  # noqa: E731
    inn = f32(innovation)
    if vasc:
        if inn is None or tuple(inn.shape) != (B, H, P):
            raise ValueError(f"innovation must be [B,H,{P}] for K={K}")
        out["debt"] = torch.empty(B, H, P, device=dev, dtype=torch.float32)
        out["arrival"] = torch.empty(B, H, P, device=dev, dtype=torch.float32)
        out["service"] = torch.empty(B, H, P, device=dev, dtype=torch.float32)
        out["gate"] = torch.empty(1, device=dev, dtype=torch.int32)
        if workspace is None:
            workspace = select_workspace(B, H, Q, K, dev)
    if want_priority:
        out["priority"] = torch.empty(B, H, Q, K, device=dev, dtype=torch.float32)
    if want_mask:
        out["mask"] = torch.empty(B, H, Q, K, device=dev, dtype=torch.uint8)
    rc = None if row_cap is None else row_cap.to(torch.int32).contiguous()
    pm = None if protected_mask is None else protected_mask.to(torch.uint8).contiguous()
    state = [f32(debt), f32(pending_arrival), f32(prev_service)]
    for t, name in zip(state, ("debt", "pending_arrival", "prev_service")):
        if t is not None and t.numel() != B * H * P:
            raise ValueError(f"{name} must hold B*H*P={B * H * P} values")
    ws_bytes = workspace.numel() if workspace is not None else 0
    _lib.call("vasc_select_blocks", s.data_ptr(), _ptr(inn), B, H, Q, K, int(mode), int(topk), _ptr(rc),
              _ptr(pm), int(bool(force_last)), int(maxc), int(sink_blocks), _ptr(state[0]),
              _ptr(state[1]), _ptr(state[2]), _ptr(out.get("debt")), _ptr(out.get("arrival")),
              _ptr(out.get("service")), _ptr(out.get("gate")), _ptr(out.get("priority")),
              _ptr(out.get("mask")), out["index"].data_ptr(), width, out["count"].data_ptr(),
              _ptr(workspace), ws_bytes, _stream())
    return out


def settle_terminal(debt, pending_arrival, service) -> torch.Tensor:
    pend = pending_arrival.float().contiguous()
    svc = service.float().contiguous()
    d = None if debt is None else debt.float().contiguous()
    out = torch.empty_like(pend)
    _lib.call("vasc_settle_terminal", _ptr(d), pend.data_ptr(), svc.data_ptr(), pend.numel(),
              out.data_ptr(), _stream())
    return out


# ----------------------------------------------------------------- kernel 3
def pack_v(v: torch.Tensor) -> torch.Tensor:
    """Packed, transposed, key-permuted V tiles ``[B,H,ceil(T/64),64,64]`` (bf16)."""
    v = _bhtd(v, "v")
    B, H, T, D = v.shape
    nkb = math.ceil(T / BLOCK_K)
    vt = torch.empty(B, H, nkb, D, BLOCK_K, device=v.device, dtype=torch.bfloat16)
    _lib.call("vasc_pack_v", v.data_ptr(), *v.stride()[:3], B, H, T, D, vt.data_ptr(), _stream())
    return vt


# ----------------------------------------------------------------- kernel 4
def block_sparse_attn(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, index: torch.Tensor,
                      count: torch.Tensor, *, scale: float | None = None, delta: bool = False,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Block-sparse attention over listed 64-key blocks; bf16 output ``[B,H,Nq,D]``."""
    q = _bhtd(q, "q")
    k = _bhtd(k, "k")
    _dev(vt, "vt")
    B, H, nq, D = q.shape
    nk = k.shape[2]
    if vt.shape != (B, H, math.ceil(nk / BLOCK_K), D, BLOCK_K):
        raise ValueError(f"vt shape {tuple(vt.shape)} does not match K {tuple(k.shape)}")
    qb = math.ceil(nq / BLOCK_Q)
    index = index.to(torch.int32).contiguous()
    count = count.to(torch.int32).contiguous()
    if index.shape[:3] != (B, H, qb) or count.shape != (B, H, qb):
        raise ValueError(f"index/count must be [B,H,{qb},W]/[B,H,{qb}]")
    o = out if out is not None else torch.empty(B, H, nq, D, device=q.device, dtype=torch.bfloat16)
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_block_sparse_attn_fwd", q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
              vt.data_ptr(), o.data_ptr(), *o.stride()[:3], B, H, nq, nk, D, index.data_ptr(),
              index.shape[-1], count.data_ptr(), int(bool(delta)), float(scale), _stream())
    return o


def dense_attn(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, *, scale: float | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Dense attention with the same MFMA kernel (every key block)."""
    q = _bhtd(q, "q")
    k = _bhtd(k, "k")
    _dev(vt, "vt")
    B, H, nq, D = q.shape
    nk = k.shape[2]
    if vt.shape != (B, H, math.ceil(nk / BLOCK_K), D, BLOCK_K):
        raise ValueError(f"vt shape {tuple(vt.shape)} does not match K {tuple(k.shape)}")
    o = out if out is not None else torch.empty(B, H, nq, D, device=q.device, dtype=torch.bfloat16)
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_dense_attn_fwd", q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
              vt.data_ptr(), o.data_ptr(), *o.stride()[:3], B, H, nq, nk, D, float(scale), _stream())
    return o
