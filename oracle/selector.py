"""CPU restatement of VASC's block selection and cross-layer memory.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

Follows ``src/sparse_vggt/utils/sparse_wrapper.py`` (``SW``) of the reference:

* ``topk_block_mask``      ``get_block_mask`` ratio/top-k branch
                           (``SW:1199-1268``) with the fill kernel's min-1
                           rule (``spas_sage_attn/utils.py:283-292``).
* ``cdf_counts``,          its cdf-threshold branch (``SW:1238-1254``):
  ``cdf_block_mask``       sequential float32 running sum over the
                           descending row, prefix count against
                           ``thr + eps``.
* ``innovation``           pair innovation of pooled values (``SW:3733-3740``).
* ``cosa_select``          ``get_cosa_value_risk_pair_debt_mask``
                           (``SW:3632-4098``) in the release ``vasc``
                           configuration: conservative arrival and debt
                           projection (``SW:1755-1769``), QK-admission service
                           reduced from the selected indices
                           (``SW:2922-2980``).
* ``selected_indices``     the selector's ``priority.topk(M, sorted=True)``
                           indices (``SW:3887-3894``).
* ``finalize``             ``finalize_cosa_value_risk_pair_debt``
                           (``SW:4101-4177``).

Arithmetic is float32 wherever the reference holds a float32 tensor; every
reduction uses the canonical orders of ``oracle/canon.py`` so the HIP select
kernels reproduce the same bits. Selection keeps the ``c`` largest priorities
with ties broken towards the lower block index (``torch.topk`` leaves tie
order unspecified).

Parity pins (``tests/test_oracle_selector.py``, ``tests/test_golden.py``):
golden vectors written by running the reference's own selector functions in
this container (``tests/golden/make_golden.py``), the invariants of the
reference's ``tests/check_selector.py`` (exact capacity, protected kept,
finite priority, memory activates, terminal settlement idempotent) and closed
forms: layer 0 priority equals the conservative arrival, uniform innovation
without saturation reduces to Top-K on the score, zero innovation selects the
first ``cap`` indices, zero debt disables the gate, brute-force Top-K on tiny
rows; the selected indices against torch's own topk on rows of distinct
priorities and a brute-force sort with ties. The cdf count is pinned against torch's own sort / cumsum /
searchsorted (the reference's primitives) on dyadic scores, where every
prefix sum is exact, and against a brute-force loop and closed forms.
"""
from __future__ import annotations

import math

import numpy as np

from .canon import FLT_MAX, FLT_MIN, chunked_sum, clamp01, clamp_min0, f32, order_key, seq_sum, wave_sum

STATE_KEY = "cosa_value_risk_pair_debt"
PENDING_KEY = "cosa_value_risk_pair_pending_arrival"
PENDING_LAYER_KEY = "cosa_value_risk_pair_pending_layer"
SERVICE_KEY = "qk_pv_service_observation"


# --------------------------------------------------------------------------
# Top-c selection with the canonical tie rule
# --------------------------------------------------------------------------
def priority_order(priority: np.ndarray) -> np.ndarray:
    """Each row's indices, largest priority first, ties in ascending index.

    Canonical form of ``priority.topk(K, sorted=True).indices``; int64.
    """
    prio = np.asarray(priority, dtype=np.float32)
    K = prio.shape[-1]
    key = order_key(prio).astype(np.uint64)
    idx = np.arange(K, dtype=np.uint64)
    composite = (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)
    return np.argsort(composite, axis=-1, kind="stable")[..., ::-1].astype(np.int64)


def selected_indices(priority: np.ndarray, M: int) -> np.ndarray:
    """The selector's ``selected_indices`` (SW:3887-3894, stored at
    SW:4024-4026): ``priority.topk(M, dim=-1, sorted=True).indices``, the M
    largest priorities of each row in descending order, ties in ascending
    index. int64 ``[..., M]``."""
    return priority_order(priority)[..., :int(M)]


def select_top(priority: np.ndarray, count: np.ndarray) -> np.ndarray:
    """Boolean mask of the ``count[...]`` largest entries of each row.

    Ties go to the lower index. ``count`` broadcasts against
    ``priority.shape[:-1]`` and is clipped to ``[0, K]``.
    """
    prio = np.asarray(priority, dtype=np.float32)
    K = prio.shape[-1]
    order = priority_order(prio)
    rank = np.empty_like(order)
    np.put_along_axis(rank, order, np.broadcast_to(np.arange(K), order.shape), axis=-1)
    c = np.clip(np.broadcast_to(np.asarray(count), prio.shape[:-1]), 0, K)
    return rank < c[..., None]


def index_lists(mask: np.ndarray, width: int | None = None):
    """Ascending index lists ``[..., width]`` (padded with -1) and counts."""
    mask = np.asarray(mask, dtype=bool)
    counts = mask.sum(-1).astype(np.int32)
    width = int(counts.max()) if width is None else int(width)
    width = max(width, 0)
    flat = mask.reshape(-1, mask.shape[-1])
    out = np.full((flat.shape[0], width), -1, dtype=np.int32)
    for r in range(flat.shape[0]):
        nz = np.flatnonzero(flat[r])
        out[r, : nz.size] = nz
    return out.reshape(mask.shape[:-1] + (width,)), counts


# --------------------------------------------------------------------------
# Top-K mode (get_block_mask)
# --------------------------------------------------------------------------
def ratio_to_topk(key_blocks: int, sparse_ratio: float) -> int:
    """``int(k_blk * (1 - sparse_ratio))`` exactly as ``SW:1226-1228``."""
    return int(key_blocks * (1 - sparse_ratio))


def topk_block_mask(score: np.ndarray, sink_blocks: int, topk: int | None = None,
                    sparse_ratio: float | None = None) -> np.ndarray:
    """``get_block_mask`` for the top-k / ratio modes (``SW:1199-1268``).

    Returns bool ``[B,H,Q,K+sink]``: the ``max(topk, 1)`` largest pooled
    scores of each row (fill kernel min-1 rule) plus ``sink`` trailing
    always-on columns.
    """
    if (topk is None) == (sparse_ratio is None):
        raise AssertionError("exactly one of topk / sparse_ratio")
    K = score.shape[-1]
    if sparse_ratio is not None:
        topk = ratio_to_topk(K, sparse_ratio)
    n = max(int(topk), 1)
    sel = select_top(score, n)
    if sink_blocks > 0:
        sink = np.ones(sel.shape[:-1] + (sink_blocks,), dtype=bool)
        sel = np.concatenate([sel, sink], axis=-1)
    return sel


def head_thresholds(cdf_threshold, H: int) -> np.ndarray:
    """Per-head float32 thresholds: ``hyperparameter_check``
    (``spas_sage_attn/utils.py:38-50``) broadcasts a number to every head and
    takes a 1-D sequence of ``H`` values as given."""
    t = np.asarray(cdf_threshold, dtype=np.float32)
    if t.ndim == 0:
        return np.full(H, t, dtype=np.float32)
    if t.ndim != 1 or t.size != H:
        raise AssertionError(f"Hyperparameter tensor must have {H} elements")
    return t


def cdf_counts(score: np.ndarray, cdf_threshold, topk: int | None = None, eps: float = 1e-5) -> np.ndarray:
    """``num_to_select`` of ``get_block_mask``'s cdf branch (``SW:1238-1254``)
    after the fill kernel's min-1 rule (``spas_sage_attn/utils.py:289``).

    Each row is ordered by descending ``order_key`` (NaN first, as torch's
    descending sort), its running float32 sum is taken strictly in that order,
    and the count is the length of the prefix whose running sum stays
    ``<= T_h`` with ``T_h = f32(f32(thr_h) + f32(eps))``. For non-negative
    scores (softmax output) the running sum never decreases and the count
    equals ``torch.searchsorted(cdf, T, right=True)``. ``topk`` (the ratio
    budget when both are given) is a lower bound; a count of 0 becomes 1.
    The reference's cumsum is torch's CUDA scan; the canonical order here is
    sequential (the two round alike except where a prefix sum lies within an
    ulp of the threshold).
    """
    s = np.asarray(score, dtype=np.float32)
    B, H, Q, K = s.shape
    T = (head_thresholds(cdf_threshold, H) + np.float32(eps)).astype(np.float32)
    key = order_key(s)
    order = np.argsort(key, axis=-1, kind="stable")[..., ::-1]
    canon = np.where(s == 0, np.float32(0.0), np.where(np.isnan(s), np.float32(np.nan), s))
    vals = np.take_along_axis(canon, order, axis=-1)
    cdf = np.cumsum(vals, axis=-1, dtype=np.float32)  # ufunc accumulate: strictly sequential
    over = ~(cdf <= T.reshape(1, H, 1, 1))
    n = np.where(over.any(-1), np.argmax(over, axis=-1), K).astype(np.int64)
    if topk is not None:
        n = np.maximum(n, int(topk))
    return np.where(n == 0, 1, n).astype(np.int32)


def cdf_block_mask(score: np.ndarray, sink_blocks: int, cdf_threshold, sparse_ratio: float | None = None,
                   eps: float = 1e-5) -> np.ndarray:
    """``get_block_mask`` with ``cdf_threshold`` (alone or with a ratio):
    the ``cdf_counts`` largest pooled scores of each row (ties to the lower
    index) plus ``sink`` trailing always-on columns."""
    K = score.shape[-1]
    topk = None if sparse_ratio is None else ratio_to_topk(K, sparse_ratio)
    sel = select_top(score, cdf_counts(score, cdf_threshold, topk, eps))
    if sink_blocks > 0:
        sel = np.concatenate([sel, np.ones(sel.shape[:-1] + (sink_blocks,), dtype=bool)], axis=-1)
    return sel


# --------------------------------------------------------------------------
# VASC selector
# --------------------------------------------------------------------------
def clean_score(score: np.ndarray) -> np.ndarray:
    """``pooled_score.float().clamp_min(0).nan_to_num_(nan=0.0)`` (SW:3685-3689)."""
    s = np.asarray(score, dtype=np.float32)
    s = np.where(np.isnan(s), np.float32(0.0), s)
    s = np.where(s > 0, s, np.float32(0.0))
    s = np.where(np.isinf(s), FLT_MAX, s)
    return s.astype(np.float32)


def clean_value(value: np.ndarray) -> np.ndarray:
    """``pooled_value.float().nan_to_num_(nan=0.0)`` (SW:3690-3694)."""
    v = np.asarray(value, dtype=np.float32)
    v = np.where(np.isnan(v), np.float32(0.0), v)
    v = np.where(np.isposinf(v), FLT_MAX, v)
    v = np.where(np.isneginf(v), -FLT_MAX, v)
    return v.astype(np.float32)


def innovation(pooled_value: np.ndarray) -> np.ndarray:
    """Pair innovation ``0.5*sqrt(mean_d (V[2p]-V[2p+1])^2)`` (SW:3733-3740).

    ``pooled_value`` ``[B,H,K,D]``; returns float32 ``[B,H,P]``, P=ceil(K/2).
    An odd tail pairs with itself (innovation 0).
    """
    v = clean_value(pooled_value)
    K, D = v.shape[-2], v.shape[-1]
    left = v[..., 0::2, :]
    right = v[..., 1::2, :]
    if right.shape[-2] != left.shape[-2]:
        right = np.concatenate([right, left[..., -1:, :]], axis=-2)
    diff = (left - right).astype(np.float32)
    sq = (diff * diff).astype(np.float32)
    mean = f32(wave_sum(sq, axis=-1) / D)
    return (np.sqrt(mean).astype(np.float32) * np.float32(0.5)).astype(np.float32)


def _pair_size(K: int) -> np.ndarray:
    P = (K + 1) // 2
    ps = np.full(P, 2.0, dtype=np.float32)
    if K % 2:
        ps[-1] = 1.0
    return ps


def conservative_arrival(score: np.ndarray, iota: np.ndarray, cap: np.ndarray):
    """Row arrival ``A`` and its pair reductions (SW:3741-3791, 1755-1769).

    Returns ``A [B,H,Q,K]``, ``a [B,H,Q,P]`` (row pair arrival),
    ``rowpair [B,H,Q]`` and the per-row risk total ``[B,H,Q]``.
    """
    s = clean_score(score)
    K = s.shape[-1]
    iota_k = np.repeat(iota, 2, axis=-1)[..., :K].astype(np.float32)
    risk = (s * iota_k[..., None, :]).astype(np.float32)
    total = f32(wave_sum(risk, axis=-1))
    capf = np.asarray(cap, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        scale = (capf / np.maximum(total, FLT_MIN)).astype(np.float32)
        proj = clamp01((risk * scale[..., None]).astype(np.float32))
    A = np.where((total > 0)[..., None], proj, np.float32(0.0)).astype(np.float32)
    P = (K + 1) // 2
    padded = np.concatenate([A, np.zeros(A.shape[:-1] + (K % 2,), np.float32)], axis=-1)
    pair_sum = (padded[..., 0::2] + padded[..., 1::2]).astype(np.float32)
    a = (pair_sum / _pair_size(K)).astype(np.float32)
    spread = np.zeros(A.shape[:-1] + (2 * P,), dtype=np.float32)
    spread[..., 0::2] = a
    rowpair = f32(wave_sum(spread[..., :K], axis=-1))
    assert a.shape[-1] == P
    return A, a, rowpair, total


def settle(debt, pending_arrival, service):
    """Ledger settlement ``U = D + Abar - Sigma`` (SW:3793-3832).

    All arrays ``[B,H,P]`` float32. Returns ``(new_debt, reflection)``.
    """
    U = ((debt + pending_arrival).astype(np.float32) - service).astype(np.float32)
    refl = clamp_min0(-U)
    return clamp_min0(U), refl


def _global_sum(x: np.ndarray) -> np.float32:
    """Sum over all B,H,P: wave sum per head, then sequential over heads."""
    x = np.asarray(x, np.float32)
    per_head = wave_sum(x.reshape(-1, x.shape[-1]), axis=-1)
    return f32(seq_sum(per_head))


def service_gate(service, reflection) -> bool:
    """Global debt gate (SW:3837-3842): useful repayment >= wasted service."""
    useful = _global_sum(clamp_min0((service - reflection).astype(np.float32)))
    wasted = _global_sum(reflection)
    consumed = _global_sum(service)
    return bool((consumed > 0) and (useful >= wasted))


def admitted_debt(debt, pair_cap):
    """Conservative debt projection (SW:3852-3859 -> 1755-1769). ``[B,H,P]``."""
    dsum = f32(wave_sum(debt, axis=-1))
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        scale = (np.asarray(pair_cap, np.float32) / np.maximum(dsum, FLT_MIN)).astype(np.float32)
        proj = clamp01((debt * scale[..., None]).astype(np.float32))
    return np.where((dsum > 0)[..., None], proj, np.float32(0.0)).astype(np.float32)


def qk_service(selected: np.ndarray, patch_blocks: int) -> np.ndarray:
    """QK-admission service per pair (SW:2922-2980): selected children per
    pair over all rows / (pair_size * Q). ``selected`` bool ``[B,H,Q,K]``.
    Returns float32 ``[B,H,P]``.
    """
    K = patch_blocks
    Q = max(selected.shape[-2], 1)
    P = (K + 1) // 2
    sel = selected[..., :K].astype(np.int64)
    if K % 2:
        sel = np.concatenate([sel, np.zeros(sel.shape[:-1] + (1,), np.int64)], axis=-1)
    counts = sel.reshape(sel.shape[:-1] + (P, 2)).sum(-1).sum(-2)
    denom = (_pair_size(K) * np.float32(Q)).astype(np.float32)
    return (counts.astype(np.float32) / denom).astype(np.float32)


def pv_execution_service(execution_map: np.ndarray, patch_blocks: int) -> np.ndarray:
    """PV-execution service per pair (``_reduce_exact_pv_execution_to_pair``,
    SW:2983-3028): executed children per pair summed over query blocks, query
    warps and the pair, over ``query_warps * pair_size`` with ``query_warps =
    Q * W``. ``execution_map`` binary ``[B,H,Q,W,K]``. Returns float32
    ``[B,H,P]``."""
    ex = np.asarray(execution_map)[..., :patch_blocks].astype(np.int64)
    if patch_blocks % 2:
        ex = np.concatenate([ex, np.zeros(ex.shape[:-1] + (1,), np.int64)], axis=-1)
    P = (patch_blocks + 1) // 2
    counts = ex.reshape(ex.shape[:-1] + (P, 2)).sum(axis=(-1, -3, -4))  # pair, warp, query block
    query_warps = execution_map.shape[-3] * execution_map.shape[-2]
    denom = (np.float32(query_warps) * _pair_size(patch_blocks)).astype(np.float32)
    return (counts.astype(np.float32) / denom).astype(np.float32)


def cosa_select(score, pooled_value, cap, *, layer_idx: int, state: dict,
                protected=None, max_capacity_hint: int | None = None,
                iota=None):
    """One layer of the VASC selector (SW:3632-4098), release configuration.

    score         float32 ``[B,H,Q,K]`` pooled probabilities.
    pooled_value  ``[B,H,K,D]`` pooled values (ignored when ``iota`` given).
    cap           int ``[B,H,Q]`` per-row QK budget (``base_mask.sum(-1)``).
    state         dict mutated in place with the reference's keys.
    protected     optional bool ``[B,H,Q,K]`` blocks forced to FLT_MAX.

    Returns ``(selected bool [B,H,Q,K], info dict)``.
    """
    s = clean_score(score)
    B, H, Q, K = s.shape
    P = (K + 1) // 2
    cap = np.broadcast_to(np.asarray(cap, dtype=np.int64), (B, H, Q))
    if max_capacity_hint is not None:
        M = min(int(max_capacity_hint), K)
    else:
        M = int(cap.max()) if cap.size else 0
    if iota is None:
        iota = innovation(pooled_value)
    A, a, rowpair, total = conservative_arrival(s, iota, cap)
    arrival = f32(chunked_sum(a, axis=-2) / Q)                   # [B,H,P]
    pair_cap = f32(wave_sum(rowpair, axis=-1) / Q)               # [B,H]

    prev = state.get(STATE_KEY)
    if prev is None or tuple(prev.shape) != (B, H, 1, P):
        debt = np.zeros((B, H, P), np.float32)
    else:
        debt = clamp_min0(np.asarray(prev, np.float32).reshape(B, H, P))
    debt_before = debt
    pending = state.get(PENDING_KEY)
    obs = state.pop(SERVICE_KEY, None)
    service_prev = np.zeros((B, H, P), np.float32)
    refl = np.zeros((B, H, P), np.float32)
    if pending is not None:
        if obs is None or not obs.get("identity_observed", False):
            raise RuntimeError("CoSA pair debt requires exact PV service identity")
        if obs.get("layer_idx") != state.get(PENDING_LAYER_KEY):
            raise RuntimeError("PV service does not match pending CoSA layer")
        service_prev = np.asarray(obs["pair_service_fraction"], np.float32).reshape(B, H, P)
        pend = np.asarray(pending, np.float32).reshape(B, H, P)
        debt, refl = settle(debt, pend, service_prev)
    gate = service_gate(service_prev, refl) if pending is not None else False
    adm = admitted_debt(debt, pair_cap)
    adm_k = np.repeat(adm, 2, axis=-1)[..., :K]
    prio = (A + adm_k[..., None, :]).astype(np.float32) if gate else A.copy()
    if protected is not None:
        prio = np.where(np.asarray(protected, bool), FLT_MAX, prio).astype(np.float32)
    count = np.minimum(cap, M)
    selected = select_top(prio, count) if M > 0 else np.zeros((B, H, Q, K), bool)
    service = qk_service(selected, K)

    state[STATE_KEY] = debt.reshape(B, H, 1, P)
    state[PENDING_KEY] = arrival.reshape(B, H, 1, P)
    state[PENDING_LAYER_KEY] = int(layer_idx)
    state[SERVICE_KEY] = {
        "layer_idx": int(layer_idx),
        "identity_observed": True,
        "service_domain": "qk_admission",
        "pair_service_fraction": service.reshape(B, H, 1, P),
    }
    state["cosa_value_risk_pair_priority"] = prio
    state["cosa_value_risk_pair_max_patch_blocks"] = int(M)
    state["cosa_value_risk_pair_selected_indices"] = selected_indices(prio, M)
    state["cosa_value_risk_pair_qk_order_priority"] = s
    info = dict(arrival=arrival, pair_cap=pair_cap, row_arrival=A, row_pair=a,
                rowpair=rowpair, total=total, gate=gate, admitted=adm,
                debt_before=debt_before, debt=debt, reflection=refl,
                service=service, priority=prio, iota=iota, count=count, M=M,
                settled=np.zeros_like(debt) if pending is None else np.asarray(pending, np.float32).reshape(B, H, P),
                consumed=service_prev, selected=selected)
    return selected, info


def routing_stats(info: dict, cap, base_mask, protected=None, counterfactual: bool = True) -> dict:
    """The selector's routing statistics (SW:4032-4096) from a ``cosa_select``
    call's ``info`` (float64 means of the float32 quantities): ledger flow of
    the settlement, gate, capacity, QK overlap with ``base_mask`` (bool
    ``[B,H,Q,K]``), budget and conservation errors and, with
    ``counterfactual``, the overlap of the current-only (row arrival) and the
    debt (arrival + admitted debt) selections."""
    debt_before = np.asarray(info["debt_before"], np.float32)
    settled = np.asarray(info.get("settled", np.zeros_like(debt_before)), np.float32)
    consumed = np.asarray(info.get("consumed", np.zeros_like(debt_before)), np.float32)
    refl = np.asarray(info["reflection"], np.float32)
    debt = np.asarray(info["debt"], np.float32)
    useful = float(clamp_min0((consumed - refl).astype(np.float32)).astype(np.float64).sum())
    wasted = float(refl.astype(np.float64).sum())
    total = float(consumed.astype(np.float64).sum())
    cap = np.asarray(cap, np.int64)
    selected = info["selected"]
    denom = np.maximum(cap, 1).astype(np.float64)
    overlap = (selected & np.asarray(base_mask, bool)).sum(-1)
    out = {
        "cosa_pair_debt_enabled": 1.0,
        "cosa_pair_service_useful_repayment": useful,
        "cosa_pair_service_wasted": wasted,
        "cosa_pair_service_utilization": useful / max(total, 1e-8) if total > 0 else 0.0,
        "cosa_pair_service_gate_debt": float(info["gate"]),
        "cosa_pair_qk_capacity": float(cap.mean()),
        "cosa_pair_arrival": float(np.asarray(info["arrival"], np.float64).sum(-1).mean()),
        "cosa_pair_innovation": float(np.asarray(info["iota"], np.float64).mean()),
        "cosa_pair_debt_before_service": float(debt_before.astype(np.float64).mean()),
        "cosa_pair_settled_arrival": float(settled.astype(np.float64).sum(-1).mean()),
        "cosa_pair_consumed_pv_service": float(consumed.astype(np.float64).sum(-1).mean()),
        "cosa_pair_admitted_debt": float(np.asarray(info["admitted"], np.float64).sum(-1).mean()),
        "cosa_pair_backlog": float(debt.astype(np.float64).sum(-1).mean()),
        "cosa_pair_qk_overlap": float((overlap / denom).mean()),
        "cosa_pair_qk_swap_fraction": float((1.0 - overlap / denom).mean()),
        "cosa_pair_budget_error": float(np.abs(selected.sum(-1) - cap).max()),
        "cosa_pair_conservation_error": float(np.abs(
            debt.astype(np.float64) - debt_before - settled + consumed - refl).max()),
    }
    if counterfactual:
        A = np.asarray(info["row_arrival"], np.float32)
        K = A.shape[-1]
        adm_k = np.repeat(np.asarray(info["admitted"], np.float32), 2, axis=-1)[..., :K]
        cur_p, debt_p = A, (A + adm_k[..., None, :]).astype(np.float32)
        if protected is not None:
            cur_p = np.where(protected, FLT_MAX, cur_p).astype(np.float32)
            debt_p = np.where(protected, FLT_MAX, debt_p).astype(np.float32)
        count = info["count"]
        both = (select_top(cur_p, count) & select_top(debt_p, count)).sum(-1)
        out["cosa_pair_current_debt_overlap"] = float((both / denom).mean())
        out["cosa_pair_history_swap_fraction"] = float((1.0 - both / denom).mean())
    return out


def finalize(state: dict) -> dict:
    """Terminal settlement (SW:4101-4177). Returns {} when nothing is pending."""
    if state is None:
        return {}
    pending = state.pop(PENDING_KEY, None)
    pending_layer = state.pop(PENDING_LAYER_KEY, None)
    if pending is None:
        return {}
    obs = state.pop(SERVICE_KEY, None)
    if obs is None or not obs.get("identity_observed", False):
        raise RuntimeError("terminal CoSA settlement requires exact PV service")
    if obs.get("layer_idx") != pending_layer:
        raise RuntimeError("terminal PV service does not match CoSA layer")
    pending = np.asarray(pending, np.float32)
    service = np.asarray(obs["pair_service_fraction"], np.float32).reshape(pending.shape)
    prev = state.get(STATE_KEY)
    if prev is None or tuple(np.shape(prev)) != tuple(pending.shape):
        prev = np.zeros_like(pending)
    else:
        prev = clamp_min0(np.asarray(prev, np.float32))
    terminal, refl = settle(prev, pending, service)
    state[STATE_KEY] = terminal
    return {
        "cosa_pair_terminal_settled": 1.0,
        "cosa_pair_terminal_layer": float(pending_layer),
        "cosa_pair_terminal_arrival": float(pending.sum(-1).mean()),
        "cosa_pair_terminal_service": float(service.sum(-1).mean()),
        "cosa_pair_terminal_backlog": float(terminal.sum(-1).mean()),
        "cosa_pair_terminal_conservation_error": float(np.abs(
            terminal.astype(np.float64) - prev - pending + service - refl).max()),
    }


# --------------------------------------------------------------------------
# block_sparse_attn_cuda selection wiring (SW:6998-7041, 7559-7770)
# --------------------------------------------------------------------------
def layer_selection(score, *, mode: str, sparse_ratio: float | None, patch_tokens: int,
                    total_tokens: int, official_mask: bool, state: dict | None = None,
                    layer_idx: int = 0, pooled_value=None, iota=None, block_k: int = 64,
                    cdf_threshold=None):
    """Final block map ``[B,H,Q,Kb+sink]`` for ``mode`` in {topk, vasc}.

    Mirrors the default branch of ``block_sparse_attn_cuda``: base map from
    ``get_block_mask`` (ratio, cdf, or both) with sink columns, the mixed-tail
    rule (forced + protected unless the official mask is requested) and, in
    vasc mode, the CoSA selector with ``hint = int(Kb*(1-s)) + [protected]``
    for the ratio alone and no hint (``M = max cap``) when a cdf threshold is
    given (``SW:7744-7750``).
    """
    Kb = score.shape[-1]
    total_blocks = math.ceil(total_tokens / block_k)
    sink = total_blocks - Kb
    mixed = patch_tokens < total_tokens and patch_tokens % block_k != 0
    if cdf_threshold is None:
        final = topk_block_mask(score, sink, sparse_ratio=sparse_ratio)
    else:
        final = cdf_block_mask(score, sink, cdf_threshold, sparse_ratio=sparse_ratio)
    force_last = mixed and not official_mask
    if force_last:
        final[..., Kb - 1] = True
    if mode == "topk":
        return final, None
    if mode != "vasc":
        raise ValueError(mode)
    protected = None
    if force_last:
        protected = np.zeros(score.shape, bool)
        protected[..., Kb - 1] = True
    cap = final[..., :Kb].sum(-1)
    hint = None if cdf_threshold is not None else ratio_to_topk(Kb, sparse_ratio) + int(protected is not None)
    sel, info = cosa_select(score, pooled_value, cap, layer_idx=layer_idx, state=state,
                            protected=protected, max_capacity_hint=hint, iota=iota)
    final = np.concatenate([sel, final[..., Kb:]], axis=-1)
    return final, info
