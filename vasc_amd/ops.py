"""Torch-facing wrappers of the C-ABI kernels (one per entry point).

Each wrapper validates shapes and dtypes, allocates outputs with torch's
caching allocator, and launches on ``torch.cuda.current_stream()``. Inputs
must be device tensors; nothing here falls back to the CPU.
"""
from __future__ import annotations

import math

import numpy as np
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
def pool_qk_max(q: torch.Tensor, k: torch.Tensor):
    """Block max pooling of Q (128 tokens) and K (64 tokens), bf16:
    ``predict_attention(pool_mode="max")``'s pooling."""
    q = _bhtd(q, "q")
    k = _bhtd(k, "k")
    B, H, nq, D = q.shape
    nk = k.shape[2]
    pq = torch.empty(B, H, math.ceil(nq / BLOCK_Q), D, device=q.device, dtype=torch.bfloat16)
    pk = torch.empty(B, H, math.ceil(nk / BLOCK_K), D, device=q.device, dtype=torch.bfloat16)
    _lib.call("vasc_pool_qk_max", q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3], B, H, nq, nk, D,
              BLOCK_Q, BLOCK_K, pq.data_ptr(), pk.data_ptr(), _stream())
    return pq, pk


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
                   round_bf16: bool = True, priority: bool = False):
    """fp32 ``softmax(bf16(bf16(pq.pk) * scale))`` over key blocks, ``[B,H,Qb,Kb]``.

    ``priority=True`` returns ``(prob, priority)`` with ``priority`` the
    VASC ledger's QK-order priority ``max(prob, 0)``, NaN -> 0, written by
    the same launch.
    """
    _dev(pooled_q, "pooled_q")
    _dev(pooled_k, "pooled_k")
    pq = pooled_q.to(torch.bfloat16).contiguous()
    pk = pooled_k.to(torch.bfloat16).contiguous()
    B, H, qb, D = pq.shape
    kb = pk.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    prob = torch.empty(B, H, qb, kb, device=pq.device, dtype=torch.float32)
    prio = torch.empty_like(prob) if priority else None
    size = _lib.load().vasc_pooled_softmax_workspace_size(B, H, qb, kb)
    ws = torch.empty(size, device=pq.device, dtype=torch.uint8) if size else None
    _lib.call("vasc_pooled_softmax", pq.data_ptr(), pk.data_ptr(), B, H, qb, kb, D, float(scale),
              int(bool(round_bf16)), prob.data_ptr(), _ptr(prio), _ptr(ws), _stream())
    return (prob, prio) if priority else prob


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


def select_workspace_region(workspace: torch.Tensor, B: int, H: int, Q: int, K: int, region: int) -> torch.Tensor:
    """A result region of the VASC selection workspace after a VASC call
    (``vasc_select_workspace_offset``): per-row totals, pair sums (float32
    ``[B,H,Q]``), capacities (int32 ``[B,H,Q]``) or the admitted debt
    (float32 ``[B,H,P]``)."""
    off = int(_lib.fn("vasc_select_workspace_offset")(B, H, Q, K, int(region)))
    if off < 0:
        raise ValueError(f"unknown workspace region {region}")
    P = (K + 1) // 2
    n, dtype = {_lib.WS_ROW_TOTAL: (B * H * Q, torch.float32), _lib.WS_ROW_PAIR_SUM: (B * H * Q, torch.float32),
                _lib.WS_ROW_CAPACITY: (B * H * Q, torch.int32), _lib.WS_ADMITTED_DEBT: (B * H * P, torch.float32)}[region]
    shape = (B, H, P) if region == _lib.WS_ADMITTED_DEBT else (B, H, Q)
    return workspace[off:off + 4 * n].view(dtype).view(shape)


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
        maxc = mc_arg = min(int(max_capacity), K)
    elif row_cap is not None:  # per-row counts, each at most max_capacity (0 = K), plus the forced tail
        mc_arg = int(max_capacity)
        maxc = min((mc_arg if mc_arg > 0 else K) + int(bool(force_last)), K)
    else:
        maxc = mc_arg = min(max(int(topk), 1) + int(bool(force_last)), K)
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
        out["workspace"] = workspace
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
              _ptr(pm), int(bool(force_last)), int(mc_arg), int(sink_blocks), _ptr(state[0]),
              _ptr(state[1]), _ptr(state[2]), _ptr(out.get("debt")), _ptr(out.get("arrival")),
              _ptr(out.get("service")), _ptr(out.get("gate")), _ptr(out.get("priority")),
              _ptr(out.get("mask")), out["index"].data_ptr(), width, out["count"].data_ptr(),
              _ptr(workspace), ws_bytes, _stream())
    return out


def cdf_counts(score: torch.Tensor, cdf_threshold, *, min_count: int = 0, force_last: bool = False,
               eps: float = 1e-5, want_base: bool = False):
    """Per-row counts of ``get_block_mask``'s cdf-threshold branch (kernel 2).

    ``cdf_threshold``: a number or ``H`` per-head values
    (``hyperparameter_check``); the kernel compares against
    ``f32(f32(thr) + f32(eps))``. Returns ``(count, base)`` int32 ``[B,H,Q]``
    (``base`` adds the forced mixed tail, ``None`` unless ``want_base``).
    """
    _dev(score, "score")
    s = score.float().contiguous()
    B, H, Q, K = s.shape
    thr = cdf_threshold.detach().float().cpu().numpy() if isinstance(cdf_threshold, torch.Tensor) else cdf_threshold
    thr = np.asarray(thr, dtype=np.float32)
    if thr.ndim == 0:
        thr = np.full(H, thr, dtype=np.float32)
    if thr.ndim != 1 or thr.size != H:
        raise ValueError(f"cdf_threshold must be a number or hold {H} values")
    T = torch.from_numpy((thr + np.float32(eps)).astype(np.float32)).to(s.device)
    count = torch.empty(B, H, Q, device=s.device, dtype=torch.int32)
    base = torch.empty_like(count) if want_base else None
    _lib.call("vasc_cdf_counts", s.data_ptr(), B, H, Q, K, T.data_ptr(), int(min_count), int(bool(force_last)),
              count.data_ptr(), _ptr(base), _stream())
    return count, base


def priority_order(priority: torch.Tensor, M: int, index: torch.Tensor | None = None,
                   count: torch.Tensor | None = None, sink: int = 0) -> torch.Tensor:
    """The selector's selected indices (kernel 2): per row the ``M`` blocks
    of largest priority, largest first, equal priorities in ascending block
    index, as ``priority.topk(M, dim=-1, sorted=True).indices``
    (SW:3887-3894). ``priority`` float32 ``[..., K]``; returns int64
    ``[..., M]``. ``index`` / ``count`` / ``sink``: the ``select_blocks``
    lists of the same selection; rows that kept exactly ``M`` patch blocks
    take them from there."""
    _dev(priority, "priority")
    p = priority.float().contiguous()
    K = p.shape[-1]
    if not 0 <= int(M) <= K:
        raise ValueError(f"M={M} outside [0, {K}]")
    out = torch.empty(p.shape[:-1] + (int(M),), device=p.device, dtype=torch.int64)
    rows = p.numel() // K if K else 0
    width = 0
    if index is not None:
        if count is None or index.dtype != torch.int32 or count.dtype != torch.int32:
            raise ValueError("index and count must be the int32 lists of select_blocks")
        if index.shape[:-1] != p.shape[:-1] or count.shape != p.shape[:-1]:
            raise ValueError("index and count must match the priority rows")
        index, count = index.contiguous(), count.contiguous()
        width = index.shape[-1]
    if rows and M:
        _lib.call("vasc_priority_order", p.data_ptr(), _ptr(index), _ptr(count), width, int(sink), rows, K, int(M),
                  out.data_ptr(), _stream())
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


def block_sparse_attn_pv(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, index: torch.Tensor,
                         count: torch.Tensor, pv_threshold, *, scale: float | None = None, delta: bool = False):
    """``block_sparse_attn`` with the PV post-cut; ``pv_threshold`` is a
    number or ``H`` values in log2 units. Returns ``(o, pv_map)`` with the
    int32 execution map ``[B, H, ceil(Nq/128)*4, ceil(Nk/64)]``."""
    q = _bhtd(q, "q")
    k = _bhtd(k, "k")
    _dev(vt, "vt")
    B, H, nq, D = q.shape
    nk = k.shape[2]
    if vt.shape != (B, H, math.ceil(nk / BLOCK_K), D, BLOCK_K):
        raise ValueError(f"vt shape {tuple(vt.shape)} does not match K {tuple(k.shape)}")
    qb, kb = math.ceil(nq / BLOCK_Q), math.ceil(nk / BLOCK_K)
    index = index.to(torch.int32).contiguous()
    count = count.to(torch.int32).contiguous()
    if index.shape[:3] != (B, H, qb) or count.shape != (B, H, qb):
        raise ValueError(f"index/count must be [B,H,{qb},W]/[B,H,{qb}]")
    thr = torch.as_tensor(pv_threshold, dtype=torch.float32).reshape(-1)
    thr = (thr.expand(H) if thr.numel() == 1 else thr).contiguous().to(q.device)
    if thr.numel() != H:
        raise ValueError(f"pv_threshold must be a number or hold {H} values")
    o = torch.empty(B, H, nq, D, device=q.device, dtype=torch.bfloat16)
    pv_map = torch.zeros(B, H, qb * 4, kb, device=q.device, dtype=torch.int32)
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_block_sparse_attn_pv_fwd", q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
              vt.data_ptr(), o.data_ptr(), *o.stride()[:3], B, H, nq, nk, D, index.data_ptr(),
              index.shape[-1], count.data_ptr(), int(bool(delta)), float(scale), thr.data_ptr(),
              pv_map.data_ptr(), _stream())
    return o, pv_map


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
    if out is not None:
        _dev(out, "out")
        if out.shape != (B, H, nq, D) or out.dtype != torch.bfloat16 or out.stride(3) != 1:
            raise ValueError(f"out must be bf16 {(B, H, nq, D)} with unit stride over D, "
                             f"got {out.dtype} {tuple(out.shape)} strides {out.stride()}")
    o = out if out is not None else torch.empty(B, H, nq, D, device=q.device, dtype=torch.bfloat16)
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_dense_attn_fwd", q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
              vt.data_ptr(), o.data_ptr(), *o.stride()[:3], B, H, nq, nk, D, float(scale), _stream())
    return o


def global_attn(q_patch: torch.Tensor, q_special: torch.Tensor | None, k: torch.Tensor, vt: torch.Tensor,
                index: torch.Tensor, count: torch.Tensor, *, scale: float | None = None):
    """Patch queries over their listed blocks and special queries over every
    key, in one launch. Returns ``(o_patch, o_special or None)`` (bf16)."""
    q_patch = _bhtd(q_patch, "q_patch")
    k = _bhtd(k, "k")
    _dev(vt, "vt")
    B, H, n_patch, D = q_patch.shape
    nk = k.shape[2]
    if vt.shape != (B, H, math.ceil(nk / BLOCK_K), D, BLOCK_K):
        raise ValueError(f"vt shape {tuple(vt.shape)} does not match K {tuple(k.shape)}")
    qb = math.ceil(n_patch / BLOCK_Q)
    index = index.to(torch.int32).contiguous()
    count = count.to(torch.int32).contiguous()
    if index.shape[:3] != (B, H, qb) or count.shape != (B, H, qb):
        raise ValueError(f"index/count must be [B,H,{qb},W]/[B,H,{qb}]")
    o_patch = torch.empty(B, H, n_patch, D, device=q_patch.device, dtype=torch.bfloat16)
    n_special = 0
    o_special = None
    qs_args = (None, 0, 0, 8)
    os_args = (None, 0, 0, 8)
    if q_special is not None and q_special.shape[2] > 0:
        q_special = _bhtd(q_special, "q_special")
        n_special = q_special.shape[2]
        o_special = torch.empty(B, H, n_special, D, device=q_patch.device, dtype=torch.bfloat16)
        qs_args = (q_special.data_ptr(), *q_special.stride()[:3])
        os_args = (o_special.data_ptr(), *o_special.stride()[:3])
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_global_attn_fwd", q_patch.data_ptr(), *q_patch.stride()[:3], *qs_args, k.data_ptr(),
              *k.stride()[:3], vt.data_ptr(), o_patch.data_ptr(), *o_patch.stride()[:3], *os_args, B, H, n_patch,
              n_special, nk, D, index.data_ptr(), index.shape[-1], count.data_ptr(), float(scale), _stream())
    return o_patch, o_special


def global_attn_tokens(q_patch: torch.Tensor, q_special: torch.Tensor | None, k: torch.Tensor, vt: torch.Tensor,
                       index: torch.Tensor, count: torch.Tensor, frames: int, tokens_per_frame: int, special: int,
                       *, scale: float | None = None) -> torch.Tensor:
    """``global_attn`` followed by ``restore_tokens`` in one launch: the
    results land on their frame-major token rows of ``[B, N*P, H*D]`` bf16."""
    q_patch = _bhtd(q_patch, "q_patch")
    k = _bhtd(k, "k")
    _dev(vt, "vt")
    B, H, n_patch, D = q_patch.shape
    N, P, S = int(frames), int(tokens_per_frame), int(special)
    nk = k.shape[2]
    if n_patch != N * (P - S) or nk != N * P:
        raise ValueError(f"q_patch/k hold {n_patch}/{nk} tokens, expected {N * (P - S)}/{N * P}")
    if k.shape[:2] != (B, H) or k.shape[3] != D:
        raise ValueError(f"k {tuple(k.shape)} does not match q_patch {tuple(q_patch.shape)}")
    if vt.shape != (B, H, math.ceil(nk / BLOCK_K), D, BLOCK_K):
        raise ValueError(f"vt shape {tuple(vt.shape)} does not match K {tuple(k.shape)}")
    qb = math.ceil(n_patch / BLOCK_Q)
    index = index.to(torch.int32).contiguous()
    count = count.to(torch.int32).contiguous()
    if index.shape[:3] != (B, H, qb) or count.shape != (B, H, qb):
        raise ValueError(f"index/count must be [B,H,{qb},W]/[B,H,{qb}]")
    qs_args = (None, 0, 0, 8)
    if S > 0:
        if q_special is None or tuple(q_special.shape) != (B, H, N * S, D):
            raise ValueError(f"q_special must be [B, H, {N * S}, {D}]")
        q_special = _bhtd(q_special, "q_special")
        qs_args = (q_special.data_ptr(), *q_special.stride()[:3])
    out = torch.empty(B, N * P, H * D, device=q_patch.device, dtype=torch.bfloat16)
    scale = D ** -0.5 if scale is None else scale
    _lib.call("vasc_global_attn_tokens_fwd", q_patch.data_ptr(), *q_patch.stride()[:3], *qs_args, k.data_ptr(),
              *k.stride()[:3], vt.data_ptr(), out.data_ptr(), B, H, N, P, S, nk, D, index.data_ptr(),
              index.shape[-1], count.data_ptr(), float(scale), _stream())
    return out


# ----------------------------------------------------------------- kernel 5
def _btht(t: torch.Tensor, name: str) -> tuple:
    """(pointer, sb, st, sh) of a bf16 ``[B,T,H,D]`` view with unit stride on D."""
    _dev(t, name)
    if t.dtype != torch.bfloat16 or t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        raise ValueError(f"{name} must be bf16 [B,T,H,D] with unit stride on D, 16-byte aligned rows")
    return t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)


def _param(t: torch.Tensor, name: str, numel: int, dtypes: tuple) -> torch.Tensor:
    """A [numel] parameter as a contiguous device tensor of one of ``dtypes``
    (converted to the first when it is none of them). Nothing is cached: the
    kernel reads the parameter's current values on every call."""
    t = t.detach()
    _dev(t, name)
    if t.numel() != numel:
        raise ValueError(f"{name} must hold {numel} values")
    if t.dtype not in dtypes:
        t = t.to(dtypes[0])
    return t.contiguous()


def residual_norm(x: torch.Tensor, y: torch.Tensor, gamma: torch.Tensor | None = None, norm=None):
    """Residual update of a pre-norm block and the next LayerNorm in one pass:
    ``x_new = bf16(x + bf16(y * gamma))`` (torch's bf16 LayerScale multiply and
    add) and, with ``norm = (weight or None, bias or None, eps)``, its
    LayerNorm over the last dimension (fp32 statistics, bf16 output).
    x, y: ``[..., dim]`` bf16 of one shape; gamma, weight, bias: ``[dim]``.
    Returns ``(x_new, normed or None)``; x is not modified."""
    _dev(x, "x")
    _dev(y, "y")
    if x.shape != y.shape:
        raise ValueError(f"x {tuple(x.shape)} and y {tuple(y.shape)} differ")
    if x.dtype != torch.bfloat16 or y.dtype != torch.bfloat16:
        raise ValueError("residual_norm computes on bf16 rows")
    dim = x.shape[-1]
    xr, yr = x.reshape(-1, dim), y.reshape(-1, dim)
    if xr.stride(-1) != 1:
        xr = xr.contiguous()
    if yr.stride(-1) != 1:
        yr = yr.contiguous()
    rows = xr.shape[0]
    keep = []

    def param(t, name):
        if t is None:
            return None
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16: the pass rounds as torch's bf16 ops on bf16 parameters")
        t = _param(t, name, dim, (torch.bfloat16,))
        keep.append(t)
        return t.data_ptr()

    xo = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    no = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16) if norm is not None else None
    w, b, eps = norm if norm is not None else (None, None, 0.0)
    _lib.call("vasc_residual_norm", xr.data_ptr(), xr.stride(0), yr.data_ptr(), yr.stride(0), param(gamma, "gamma"),
              param(w, "norm weight"), param(b, "norm bias"), float(eps), xo.data_ptr(), dim,
              no.data_ptr() if no is not None else None, dim, rows, dim, _stream())
    return xo, no


def _layout_args(B: int, T: int, D: int, q_norm, k_norm, pos, rope_tables) -> tuple[list, tuple]:
    """The norm and rotary arguments of the layout entry points:
    ``(tensors to keep alive, (q norm x4, k norm x4, rope x6))``."""
    keep = []

    def norm_args(nrm, name):
        if nrm is None:
            return (None, None, 0.0, 0)
        w, b, eps = nrm
        given = [t for t in (w, b) if t is not None]
        # both parameters in one dtype the kernel reads directly: bf16 (2) or float32 (1)
        kind = 2 if given and all(t.dtype == torch.bfloat16 for t in given) else 1
        out = []
        for t in (w, b):
            if t is None:
                out.append(None)
            else:
                t = _param(t, f"{name} parameters", D, (torch.bfloat16,) if kind == 2 else (torch.float32,))
                keep.append(t)
                out.append(t.data_ptr())
        return (out[0], out[1], float(eps), kind)

    rope = (None, 0, 2, None, None, 0)
    if pos is not None:
        if rope_tables is None:
            raise ValueError("rope_tables are required with pos")
        _dev(pos, "pos")
        pos32 = pos.to(torch.int32)
        if pos32.dim() == 2:
            pos32 = pos32.unsqueeze(0)
        if pos32.shape[-2:] != (T, 2) or pos32.stride(-1) != 1:
            pos32 = pos32.reshape(-1, T, 2).contiguous()
        if pos32.dim() != 3 or pos32.shape[0] not in (1, B):
            raise ValueError(f"pos must be [{B} or 1, {T}, 2], got {tuple(pos.shape)}")
        cos, sin = (t.float().contiguous() for t in rope_tables)
        if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D // 4:
            raise ValueError(f"rope tables must be [n, {D // 4}]")
        keep += [pos32, cos, sin]
        rope = (pos32.data_ptr(), pos32.stride(0) if pos32.shape[0] > 1 else 0, pos32.stride(1), cos.data_ptr(),
                sin.data_ptr(), cos.shape[0])
    return keep, (*norm_args(q_norm, "q_norm"), *norm_args(k_norm, "k_norm"), *rope)


def pack_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None, frames: int, tokens_per_frame: int,
             special: int, *, q_norm=None, k_norm=None, pos: torch.Tensor | None = None,
             rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Frame-major ``[B,T,H,D]`` q/k/v views -> ``(q_patch, q_special, k, v)``
    in the global layer's ``[patch; special]`` order, ``[B,H,*,D]`` bf16.
    ``v=None`` packs only q and k (the returned v is None).

    ``q_norm`` / ``k_norm``: ``(weight or None, bias or None, eps)`` of a
    per-head LayerNorm, or None. ``pos`` int ``[B,T,2]`` (row, column) with
    ``rope_tables = (cos, sin)`` float32 ``[n, D/4]``: 2D rotary embedding.
    """
    B, T, H, D = q.shape
    N, P, S = int(frames), int(tokens_per_frame), int(special)
    if N * P != T or k.shape != q.shape or (v is not None and v.shape != q.shape):
        raise ValueError(f"q/k/v must be [B,{N}*{P},H,D], got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{None if v is None else tuple(v.shape)}")
    dev = q.device
    qp = torch.empty(B, H, N * (P - S), D, device=dev, dtype=torch.bfloat16)
    qs = torch.empty(B, H, N * S, D, device=dev, dtype=torch.bfloat16)
    ko = torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16)
    vo = None if v is None else torch.empty(B, H, T, D, device=dev, dtype=torch.bfloat16)
    keep, args = _layout_args(B, T, D, q_norm, k_norm, pos, rope_tables)
    vsrc = (None, 0, 0, 0) if v is None else _btht(v, "v")
    _lib.call("vasc_pack_qkv", *_btht(q, "q"), *_btht(k, "k"), *vsrc, B, H, N, P, S, D, *args,
              qp.data_ptr(), qs.data_ptr(), ko.data_ptr(), _ptr(vo), _stream())
    del keep
    return qp, (qs if S else None), ko, vo


def pack_global(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, frames: int, tokens_per_frame: int,
                special: int, *, q_norm=None, k_norm=None, pos: torch.Tensor | None = None,
                rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None, innovation: bool = True,
                pooled_v: bool = False):
    """``pack_qkv`` with V packed straight into attention tiles and the
    block-mean pooling of the patch tokens in the same pass.

    Returns ``(q_patch, q_special, k, vt, pooled_q, pooled_k, innovation,
    pooled_v)``: ``q_patch`` / ``q_special`` / ``k`` as ``pack_qkv`` (bit
    for bit), ``vt`` as ``pack_v`` of the packed V, ``pooled_q`` / ``pooled_k``
    as ``pool_qkv(q_patch, k[:, :, :Np])``, ``innovation`` (or None) the pair
    innovation of the patch values' block means, ``pooled_v`` (or None) those
    means. Requires at least one patch token per frame.
    """
    B, T, H, D = q.shape
    N, P, S = int(frames), int(tokens_per_frame), int(special)
    if N * P != T or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q/k/v must be [B,{N}*{P},H,D], got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not 0 <= S < P:
        raise ValueError(f"frames of {P} tokens need at least one patch token (special={S})")
    dev = q.device
    n_patch = N * (P - S)
    kb = math.ceil(n_patch / BLOCK_K)
    bf = dict(device=dev, dtype=torch.bfloat16)
    qp = torch.empty(B, H, n_patch, D, **bf)
    qs = torch.empty(B, H, N * S, D, **bf)
    ko = torch.empty(B, H, T, D, **bf)
    vt = torch.empty(B, H, math.ceil(T / BLOCK_K), D, BLOCK_K, **bf)
    pq = torch.empty(B, H, math.ceil(n_patch / BLOCK_Q), D, **bf)
    pk = torch.empty(B, H, kb, D, **bf)
    pv = torch.empty(B, H, kb, D, **bf) if pooled_v else None
    inn = torch.empty(B, H, (kb + 1) // 2, device=dev, dtype=torch.float32) if innovation else None
    keep, args = _layout_args(B, T, D, q_norm, k_norm, pos, rope_tables)
    _lib.call("vasc_pack_global", *_btht(q, "q"), *_btht(k, "k"), *_btht(v, "v"), B, H, N, P, S, D, *args,
              qp.data_ptr(), qs.data_ptr(), ko.data_ptr(), vt.data_ptr(), pq.data_ptr(), pk.data_ptr(), _ptr(pv),
              _ptr(inn), _stream())
    del keep
    return qp, (qs if S else None), ko, vt, pq, pk, inn, pv


def restore_tokens(x_patch: torch.Tensor, x_special: torch.Tensor | None, frames: int, tokens_per_frame: int,
                   special: int) -> torch.Tensor:
    """``[B,H,Np,D]`` + ``[B,H,Ns,D]`` -> frame-major ``[B,T,H*D]`` (bf16)."""
    x_patch = _bhtd(x_patch, "x_patch")
    B, H, n_patch, D = x_patch.shape
    N, P, S = int(frames), int(tokens_per_frame), int(special)
    if n_patch != N * (P - S):
        raise ValueError(f"x_patch holds {n_patch} tokens, expected {N * (P - S)}")
    xs = (None, 0, 0, 8)
    if S:
        if x_special is None or x_special.shape[2] != N * S:
            raise ValueError(f"x_special must hold {N * S} tokens")
        x_special = _bhtd(x_special, "x_special")
        xs = (x_special.data_ptr(), *x_special.stride()[:3])
    out = torch.empty(B, N * P, H * D, device=x_patch.device, dtype=torch.bfloat16)
    _lib.call("vasc_restore_tokens", x_patch.data_ptr(), *x_patch.stride()[:3], *xs, B, H, N, P, S, D,
              out.data_ptr(), _stream())
    return out
