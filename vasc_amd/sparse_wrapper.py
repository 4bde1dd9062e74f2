"""Drop-in sparse-attention operator API (GPU only).

Mirrors the operator surface of the reference's
``src/sparse_vggt/utils/sparse_wrapper.py`` (``SW``) for the release modes:

* ``check_sparse_mode`` / ``check_sparse_mode_three_type`` (SW:1143-1196)
* ``get_block_mask`` (SW:1199-1268), ties to the lower block index
* ``get_cosa_value_risk_pair_debt_mask`` (SW:3632-4098) and
  ``finalize_cosa_value_risk_pair_debt`` (SW:4101-4177) on the same
  ``routing_state`` dict keys
* ``block_sparse_attn_cuda`` (SW:6868-8245): selection by the environment's
  mode switch (``vasc``/``topk``), mixed-tail and sink rules, V pack and the
  bf16 MFMA block-sparse attention kernel
* ``block_map_lut`` (``spas_sage_attn/utils.py:54-87``) and its inverse

Every function runs the HIP kernels of ``libvasc_hip.so``; CPU tensors are
rejected. Documented differences from the reference: attention computes in
bf16 with fp32 accumulation (the reference quantises Q/K to int8 and P to
fp16); M (``cosa_value_risk_pair_max_patch_blocks``) is the capacity hint with a
ratio, as in the reference, and ``max(topk, 1) + force_last`` with an
explicit ``topk`` where the reference reads the largest row capacity back to
the host (equal unless every row already keeps the mixed-tail block); ties in
the selection and in ``routing_state["cosa_value_risk_pair_selected_indices"]``
(``priority.topk(M, sorted=True).indices``, int64) go to the lower block
index (``torch.topk`` leaves them unspecified).
"""
from __future__ import annotations

import math
import os

import torch

from . import _lib, ops
from .launcher import pv_threshold_active, resolve_pv_threshold, routing_config

KBLK = 64
STATE_KEY = "cosa_value_risk_pair_debt"
PENDING_KEY = "cosa_value_risk_pair_pending_arrival"
PENDING_LAYER_KEY = "cosa_value_risk_pair_pending_layer"
SERVICE_KEY = "qk_pv_service_observation"
_PV_SERVICE_PENDING = "_vasc_pv_execution_service"  # service awaiting the attention launch

# Research keyword arguments of block_sparse_attn_cuda (SW:6868-6971) with the
# values the release modes pass; any other value selects a research router
# that this build does not implement.
_RESEARCH_DEFAULTS = {
    "use_radial_layerwise": False, "num_frames": None, "tokens_per_frame": None, "decay_factor": 1.0,
    "dense_neighbor": 1, "layer_sparsity_ratios": None, "use_distance_routed": False,
    "route_frame_threshold": 4, "use_covariance_aware_importance": False, "covariance_weight": 0.5,
    "covariance_eps": 1e-8, "key_block_variance": None, "use_adaptive_slit_routing": False,
    "adaptive_slit_temporal_window": 10, "adaptive_slit_stable_quantile": 0.6,
    "adaptive_slit_change_quantile": 0.7, "adaptive_slit_narrow_width": 1, "adaptive_slit_base_width": 2,
    "adaptive_slit_expand_width": 4, "use_soft_geometry_routing": False, "use_preview_adaptive_routing": False,
    "use_dual_path_routing": False, "use_layerwise_hybrid_routing": False,
    "use_local_layerwise_hybrid_routing": False, "use_coverage_layerwise_routing": False,
    "use_persistent_view_graph_routing": False, "analyze_importance_blocks": False,
    "analyze_block_selection": False,
}
# Routing knobs that only matter when their router is enabled above.
_INERT_WITHOUT_ROUTER = ("preview_", "dual_path_", "hybrid_", "mid_frame_", "view_graph_", "core_frame_",
                         "transition_frame_", "geometry_", "decay_gamma", "frame_normalize", "distance_calibrate",
                         "entropy_adaptive", "head_adaptive")


def check_sparse_mode(sparse_ratio, cdf_threshold):
    """Exactly one of: ratio, cdf, ratio + cdf (SW:1143-1166)."""
    use_ratio, use_cdf = sparse_ratio is not None, cdf_threshold is not None
    assert (use_ratio and not use_cdf) + (use_cdf and not use_ratio) + (use_ratio and use_cdf) == 1, \
        f"Current: {sparse_ratio=}, {cdf_threshold=}"


def check_sparse_mode_three_type(topk, sparse_ratio, cdf_threshold):
    """Exactly one of: topk, ratio, cdf, ratio + cdf (SW:1169-1196)."""
    t, r, c = topk is not None, sparse_ratio is not None, cdf_threshold is not None
    modes = (t and not r and not c) + (not t and r and not c) + (not t and not r and c) + (r and c and not t)
    assert modes == 1, f"Current: {topk=}, {sparse_ratio=}, {cdf_threshold=}"


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (this operator has no CPU path)")


def _budget(key_blocks: int, topk, sparse_ratio, cdf_threshold) -> int | None:
    """The uniform budget ``int(Kb*(1-s))`` or ``topk`` (SW:1224-1235);
    ``None`` for the cdf threshold alone."""
    check_sparse_mode_three_type(topk, sparse_ratio, cdf_threshold)
    if sparse_ratio is not None:
        assert 0 <= sparse_ratio <= 1
        topk = int(key_blocks * (1 - sparse_ratio))
    if topk is not None:
        assert 0 <= topk <= key_blocks
    if cdf_threshold is not None:
        thr = cdf_threshold.detach().cpu() if isinstance(cdf_threshold, torch.Tensor) else cdf_threshold
        assert bool((torch.as_tensor(thr) >= 0).all() and (torch.as_tensor(thr) <= 1).all())
    return None if topk is None else int(topk)


def get_block_mask(pooled_score: torch.Tensor, sink_blocks: int, topk: int | None = None,
                   sparse_ratio: float | None = None, cdf_threshold: float | None = None,
                   eps: float = 1e-5) -> torch.Tensor:
    """Block map with ``sink_blocks`` trailing always-on columns (SW:1199-1268).

    Returns bool ``[B,H,Q,K+sink]`` with ``max(topk,1)`` patch blocks per row,
    or with a cdf threshold the per-row count of ``ops.cdf_counts`` (at least
    the ratio budget when both are given).
    """
    _require_gpu(pooled_score, "pooled_score")
    B, H, Q, K = pooled_score.shape
    assert 0 <= sink_blocks <= K
    t = _budget(K, topk, sparse_ratio, cdf_threshold)
    if cdf_threshold is not None:
        count, _ = ops.cdf_counts(pooled_score, cdf_threshold, min_count=t or 0, eps=eps)
        out = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=0, row_cap=count, want_mask=True)
    else:
        out = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=t, want_mask=True)
    mask = out["mask"].bool()
    if sink_blocks > 0:
        mask = torch.cat([mask, mask.new_ones(B, H, Q, sink_blocks)], dim=-1)
    return mask


def block_map_lut(block_map: torch.Tensor):
    """Delta-encoded LUT and counts of a bool block map (utils.py:54-87)."""
    m = block_map.bool()
    K = m.shape[-1]
    pos = torch.arange(K, device=m.device, dtype=torch.int32).expand_as(m)
    key = torch.where(m, pos, torch.full_like(pos, K))
    idx = torch.sort(key, dim=-1).values
    count = m.sum(-1, dtype=torch.int32)
    delta = torch.diff(idx, dim=-1, prepend=torch.zeros_like(idx[..., :1]))
    valid = torch.arange(K, device=m.device).view(*([1] * (m.dim() - 1)), K) < count.unsqueeze(-1)
    return torch.where(valid, delta, torch.zeros_like(delta)).to(torch.int32), count


def _ledger_inputs(routing_state: dict, B: int, H: int, P: int):
    """Debt, pending arrival and service of the previous layer (SW:3793-3832)."""
    shape = (B, H, 1, P)
    prev = routing_state.get(STATE_KEY)
    debt = prev if (prev is not None and tuple(prev.shape) == shape) else None
    pending = routing_state.get(PENDING_KEY)
    obs = routing_state.pop(SERVICE_KEY, None)
    service = None
    if pending is not None:
        if obs is None or not obs.get("identity_observed", False):
            raise RuntimeError("CoSA pair debt requires exact PV service identity")
        if obs.get("layer_idx") != routing_state.get(PENDING_LAYER_KEY):
            raise RuntimeError("PV service does not match pending CoSA layer")
        if "pair_service_fraction" not in obs:
            raise RuntimeError("PV service observation carries no pair service fraction")
        service = obs["pair_service_fraction"]
        if tuple(service.shape) != shape:
            raise RuntimeError("PV service changed the stable pair layout")
        if tuple(pending.shape) != shape:
            raise RuntimeError("pending arrival changed the stable pair layout")
    return debt, pending, service


def _service_domain() -> str:
    """``SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN`` (SW:3996-4000; default pv_execution)."""
    domain = os.environ.get("SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN", "pv_execution").lower()
    if domain not in ("pv_execution", "qk_admission"):
        raise ValueError("unsupported CoSA debt service domain")
    return domain


def _ledger_outputs(routing_state: dict, out: dict, score: torch.Tensor, layer_idx: int, M: int,
                    domain: str = "qk_admission", priority: torch.Tensor | None = None, sink: int = 0) -> None:
    """State writes of the selector (SW:3990-4025). In the QK-admission domain
    the service observation is recorded here; in the PV-execution domain the
    attention launch records it (``_record_pv_execution``). ``out`` carries
    the execution priority; the selected indices are its top ``M`` in
    priority order. ``priority``: the cleaned score when the pooled softmax
    already wrote it."""
    B, H, Q, K = score.shape
    P = (K + 1) // 2
    routing_state[STATE_KEY] = out["debt"].view(B, H, 1, P)
    routing_state[PENDING_KEY] = out["arrival"].view(B, H, 1, P)
    routing_state[PENDING_LAYER_KEY] = int(layer_idx)
    routing_state.pop(_PV_SERVICE_PENDING, None)
    if domain == "qk_admission":
        routing_state[SERVICE_KEY] = {
            "layer_idx": int(layer_idx),
            "identity_observed": True,
            "service_domain": "qk_admission",
            "pair_service_fraction": out["service"].view(B, H, 1, P),
        }
    else:
        routing_state[_PV_SERVICE_PENDING] = (int(layer_idx), out["service"].view(B, H, 1, P))
    routing_state["cosa_value_risk_pair_priority"] = out["priority"]
    routing_state["cosa_value_risk_pair_max_patch_blocks"] = int(M)
    routing_state["cosa_value_risk_pair_selected_indices"] = ops.priority_order(out["priority"], M, out["index"],
                                                                                out["count"], sink)
    # clamp_min(0) then NaN -> 0, as the reference's score (SW:3680-3684), in one pass
    if priority is None:
        sf = score.float()
        priority = torch.where(sf > 0, sf, 0.0)
    routing_state["cosa_value_risk_pair_qk_order_priority"] = priority


def _pv_execution_service(pv_map: torch.Tensor, patch_blocks: int) -> torch.Tensor:
    """``_reduce_exact_pv_execution_to_pair`` (SW:2983-3028) of the kernel's
    execution map ``[B, H, Qb*4, Kb]``: executed children per pair summed over
    query blocks, waves and the pair (exact integers), over
    ``float(Qb*4) * pair_size``. Returns float32 ``[B, H, 1, P]``."""
    B, H, QW, _ = pv_map.shape
    ex = pv_map[..., :patch_blocks]
    if patch_blocks % 2:
        ex = torch.nn.functional.pad(ex, (0, 1))
    P = (patch_blocks + 1) // 2
    counts = ex.reshape(B, H, QW, P, 2).sum(dim=(2, 4), dtype=torch.int64)
    pair_size = torch.full((P,), 2.0, device=pv_map.device, dtype=torch.float32)
    if patch_blocks % 2:
        pair_size[-1] = 1.0
    denom = torch.tensor(float(QW), device=pv_map.device, dtype=torch.float32) * pair_size
    return (counts.to(torch.float32) / denom).view(B, H, 1, P)


def _record_pv_execution(routing_state: dict | None, pv_map: torch.Tensor | None = None,
                         patch_blocks: int | None = None) -> None:
    """PV-execution service of the layer just attended (SW:8055-8217 with
    ``_reduce_exact_pv_execution_to_pair``, SW:2983-3028).

    With the PV post-cut (``pv_map`` given) the service is reduced from the
    kernel's execution map. At the inert threshold (1e10) every listed block
    runs its PV product in each of the four 32-row query waves of its 128-row
    block: the exact reduction ``(4 * count) / (4 * Q * pair_size)`` then
    divides the same integers as the QK-admission fraction
    ``count / (Q * pair_size)`` written by the select kernel, so that fraction
    is recorded as is.
    """
    if routing_state is None:
        return
    pending = routing_state.pop(_PV_SERVICE_PENDING, None)
    if pending is None:
        return
    layer_idx, service = pending
    if pv_map is not None:
        service = _pv_execution_service(pv_map, patch_blocks)
    routing_state[SERVICE_KEY] = {
        "layer_idx": int(layer_idx),
        "identity_observed": True,
        "pair_service_fraction": service,
    }


def _pv_threshold(key: torch.Tensor, layer_idx: int) -> float | None:
    """The PV post-cut threshold of this layer (SW:7008-7027), or None when
    it is inert (1e10, or the layer is not in QK_PV_ACTIVE_LAYERS)."""
    cfg = routing_config()
    thr = resolve_pv_threshold(cfg.pv_threshold, key.shape[-2])
    if not pv_threshold_active(cfg.pv_active_layers, layer_idx) or thr >= 1e10:
        return None
    return thr


def _counterfactual_stats() -> bool:
    """SPARSE_VGGT_COSA_COUNTERFACTUAL_STATS (on unless set off, SW:3909-3912)."""
    return os.environ.get("SPARSE_VGGT_COSA_COUNTERFACTUAL_STATS", "1").lower() in {"1", "true", "yes", "on"}


def _routing_stats(score: torch.Tensor, out: dict, cap: torch.Tensor, base_mask: torch.Tensor, ledger_in: tuple,
                   innovation: torch.Tensor, protected_mask: torch.Tensor | None, M: int) -> dict:
    """The selector's routing statistics (SW:4032-4096) from the kernel's
    outputs: ledger flow of the settlement (previous debt, settled arrival,
    consumed service, reflection), the service gate, capacities, the QK
    overlap with the base map and, with counterfactual statistics on (the
    reference's default), the overlap of the current-only and debt
    selections. The admitted debt is read back from the selection workspace.
    Every value is a 0-d float32 tensor on the device."""
    B, H, P = out["debt"].shape
    Q, K = score.shape[-2:]
    debt_in, pending, service = ledger_in
    zeros = torch.zeros(B, H, P, device=score.device, dtype=torch.float32)
    prev_before = zeros if debt_in is None else debt_in.float().reshape(B, H, P).clamp_min(0.0)
    settled = zeros if pending is None else pending.float().reshape(B, H, P)
    consumed = zeros if pending is None else service.float().reshape(B, H, P)
    reflection = zeros if pending is None else (-((prev_before + settled) - consumed)).clamp_min(0.0)
    previous = out["debt"]
    useful = (consumed - reflection).clamp_min(0.0).sum()
    wasted = reflection.sum()
    consumed_total = consumed.sum()
    utilization = torch.where(consumed_total > 0, useful / consumed_total.clamp_min(1e-8),
                              torch.zeros_like(consumed_total))
    admitted = ops.select_workspace_region(out["workspace"], B, H, Q, K, _lib.WS_ADMITTED_DEBT)
    selected = out["mask"].bool()
    denominator = cap.clamp_min(1).float()
    overlap = (selected & base_mask).sum(dim=-1).float()
    stats = {
        "cosa_pair_debt_enabled": torch.ones((), device=score.device),
        "cosa_pair_service_useful_repayment": useful,
        "cosa_pair_service_wasted": wasted,
        "cosa_pair_service_utilization": utilization,
        "cosa_pair_service_gate_debt": out["gate"].float().view(()),
        "cosa_pair_qk_capacity": cap.float().mean(),
        "cosa_pair_arrival": out["arrival"].sum(dim=-1).mean(),
        "cosa_pair_innovation": innovation.float().mean(),
        "cosa_pair_debt_before_service": prev_before.mean(),
        "cosa_pair_settled_arrival": settled.sum(dim=-1).mean(),
        "cosa_pair_consumed_pv_service": consumed.sum(dim=-1).mean(),
        "cosa_pair_admitted_debt": admitted.sum(dim=-1).mean(),
        "cosa_pair_backlog": previous.sum(dim=-1).mean(),
        "cosa_pair_qk_overlap": (overlap / denominator).mean(),
        "cosa_pair_qk_swap_fraction": (1.0 - overlap / denominator).mean(),
        "cosa_pair_budget_error": (selected.sum(dim=-1) - cap).abs().amax().float(),
        "cosa_pair_conservation_error": (previous - prev_before - settled + consumed - reflection).abs().amax(),
    }
    if _counterfactual_stats():
        # current-only selection: the same arrival with no ledger (the gate
        # stays closed, so the execution priority is the current priority)
        cur = ops.select_blocks(score, mode=_lib.MODE_VASC, topk=0, innovation=innovation, row_cap=cap,
                                protected_mask=protected_mask, max_capacity=M, want_mask=True, want_priority=True)
        adm_k = admitted.repeat_interleave(2, dim=-1)[..., :K].unsqueeze(-2)
        debt_priority = cur["priority"] + adm_k
        if protected_mask is not None:
            debt_priority = debt_priority.masked_fill(protected_mask.bool(), torch.finfo(torch.float32).max)
        deb = ops.select_blocks(debt_priority, mode=_lib.MODE_TOPK, topk=0, row_cap=torch.clamp(cap, max=M),
                                max_capacity=M, want_mask=True)
        both = (cur["mask"].bool() & deb["mask"].bool()).sum(dim=-1).float()
        stats["cosa_pair_current_debt_overlap"] = (both / denominator).mean()
        stats["cosa_pair_history_swap_fraction"] = (1.0 - both / denominator).mean()
    return stats


def get_cosa_value_risk_pair_debt_mask(pooled_score: torch.Tensor, pooled_value: torch.Tensor | None,
                                       base_mask: torch.Tensor, *, layer_idx: int, routing_state: dict | None,
                                       stats_store: dict | None = None, protected_mask: torch.Tensor | None = None,
                                       max_capacity_hint: int | None = None, fp32_projection: bool = False,
                                       risk_safe_observer: bool = False, raw_value: torch.Tensor | None = None,
                                       value_block_size: int = 64) -> torch.Tensor:
    """VASC value-risk pair-debt selection of one layer (SW:3632-4098).

    Returns the bool support ``[B,H,Q,K]`` with exactly
    ``min(base_mask.sum(-1), M)`` blocks per row and updates
    ``routing_state`` in place. Arithmetic is float32 with the conservative
    projections of the release configuration (``fp32_projection`` has no
    further effect there).
    """
    if pooled_score.ndim != 4 or base_mask.shape != pooled_score.shape:
        raise ValueError("CoSA pair debt requires matching [B,H,Q,K] scores")
    if pooled_value is None and raw_value is None:
        raise ValueError("CoSA pair debt requires pooled or raw values")
    if pooled_value is not None and pooled_value.ndim != 4:
        raise ValueError("CoSA pair debt requires pooled [B,H,K,D] values")
    if pooled_value is not None and pooled_value.shape[:2] != pooled_score.shape[:2]:
        raise ValueError("pooled score/value batch and head dimensions differ")
    if pooled_value is not None and pooled_value.shape[-2] != pooled_score.shape[-1]:
        raise ValueError("pooled score/value key layouts differ")
    if raw_value is not None and raw_value.shape[:2] != pooled_score.shape[:2]:
        raise ValueError("raw value batch and head dimensions differ")
    if base_mask.dtype != torch.bool:
        raise ValueError("base_mask must be boolean")
    if layer_idx < 0:
        raise ValueError("layer_idx must be non-negative")
    if routing_state is None:
        raise ValueError("CoSA pair debt requires routing_state")
    if protected_mask is not None and protected_mask.shape != base_mask.shape:
        raise ValueError("protected mask must match the QK support")
    if max_capacity_hint is not None and max_capacity_hint < 0:
        raise ValueError("max capacity hint must be non-negative")
    if risk_safe_observer:
        raise NotImplementedError("the risk-safe observer is a research diagnostic and is not built")
    _require_gpu(pooled_score, "pooled_score")
    B, H, Q, K = pooled_score.shape
    P = (K + 1) // 2
    cap = base_mask.sum(-1, dtype=torch.int32)
    M = min(int(max_capacity_hint), K) if max_capacity_hint is not None else int(cap.max().item()) if cap.numel() else 0
    if stats_store is not None and bool((cap > M).any()):
        raise RuntimeError("capacity hint is smaller than the QK budget")
    if pooled_value is not None:
        innovation = ops.pair_innovation(pooled_value)
    else:
        if value_block_size != KBLK:
            raise NotImplementedError("value pooling is built for 64-token blocks")
        _, _, _, innovation = ops.pool_qkv(v=raw_value)
        if innovation.shape[-1] != P:
            raise RuntimeError("fused value pooling changed the QK block layout")
    debt, pending, service = _ledger_inputs(routing_state, B, H, P)
    out = ops.select_blocks(pooled_score, mode=_lib.MODE_VASC, topk=0, innovation=innovation, row_cap=cap,
                            protected_mask=protected_mask, max_capacity=M, debt=debt, pending_arrival=pending,
                            prev_service=service, want_mask=True, want_priority=True)
    _ledger_outputs(routing_state, out, pooled_score, layer_idx, M, _service_domain())
    if stats_store is not None:
        stats_store.update(_routing_stats(pooled_score, out, cap, base_mask, (debt, pending, service), innovation,
                                          protected_mask, M))
    return out["mask"].bool()


def finalize_cosa_value_risk_pair_debt(routing_state: dict | None, *, stats_store: dict | None = None) -> dict:
    """Settle the last layer's service into the ledger (SW:4101-4177).

    Returns the terminal statistics, or ``{}`` when nothing is pending (so a
    second call returns ``{}``).
    """
    if routing_state is None:
        return {}
    pending = routing_state.pop(PENDING_KEY, None)
    pending_layer = routing_state.pop(PENDING_LAYER_KEY, None)
    if pending is None:
        return {}
    obs = routing_state.pop(SERVICE_KEY, None)
    if obs is None or not obs.get("identity_observed", False):
        raise RuntimeError("terminal CoSA settlement requires exact PV service")
    if obs.get("layer_idx") != pending_layer:
        raise RuntimeError("terminal PV service does not match CoSA layer")
    if "pair_service_fraction" not in obs:
        raise RuntimeError("PV service observation carries no pair service fraction")
    service = obs["pair_service_fraction"]
    prev = routing_state.get(STATE_KEY)
    if prev is not None and tuple(prev.shape) != tuple(pending.shape):
        prev = None
    terminal = ops.settle_terminal(prev, pending, service).view(pending.shape)
    routing_state[STATE_KEY] = terminal
    dev = terminal.device
    previous = torch.zeros_like(pending) if prev is None else prev.float().clamp_min(0.0)
    reflection = (-((previous + pending) - service)).clamp_min(0.0)
    stats = {
        "cosa_pair_terminal_settled": torch.tensor(1.0, device=dev),
        "cosa_pair_terminal_layer": torch.tensor(float(pending_layer), device=dev),
        "cosa_pair_terminal_arrival": pending.sum(dim=-1).mean(),
        "cosa_pair_terminal_service": service.sum(dim=-1).mean(),
        "cosa_pair_terminal_backlog": terminal.sum(dim=-1).mean(),
        "cosa_pair_terminal_conservation_error": (terminal - previous - pending + service - reflection).abs().amax(),
    }
    if stats_store is not None:
        stats_store.update(stats)
    return stats


def _check_research_kwargs(kwargs: dict) -> None:
    for name, value in kwargs.items():
        if name in _RESEARCH_DEFAULTS:
            default = _RESEARCH_DEFAULTS[name]
            same = value is default or (value == default if not isinstance(value, torch.Tensor) else False)
            if not same:
                raise NotImplementedError(f"{name}={value!r} selects a research router that is not built")
        elif name.startswith(_INERT_WITHOUT_ROUTER):
            continue
        else:
            raise TypeError(f"block_sparse_attn_cuda() got an unexpected keyword argument {name!r}")


def _select_for_layer(key: torch.Tensor, value: torch.Tensor, pooled_score: torch.Tensor, topk, sparse_ratio,
                      cdf_threshold, layer_idx: int, routing_stats_store, routing_state, num_patch_tokens,
                      research: dict, innovation: torch.Tensor | None = None,
                      priority: torch.Tensor | None = None):
    """Mode switch, budget, mixed-tail and sink rules and kernel 2 of
    block_sparse_attn_cuda (SW:6998-7041, 7559-7770). Returns the selection
    and the total key-block count. ``innovation``: the pair innovation of
    the patch values when the caller pooled them already; ``priority``: the
    cleaned score when the caller's softmax wrote it."""
    _check_research_kwargs(research)
    for t, name in ((key, "key"), (value, "value"), (pooled_score, "pooled_score")):
        if t is not None:
            _require_gpu(t, name)
    cfg = routing_config()
    Tk = key.shape[-2]
    orig_kblk = pooled_score.shape[-1]
    total_kblk = math.ceil(Tk / KBLK)
    sink = total_kblk - orig_kblk
    if sink < 0:
        raise ValueError("pooled_score has more key blocks than the keys")
    t = _budget(orig_kblk, topk, sparse_ratio, cdf_threshold)
    mixed = num_patch_tokens is not None and num_patch_tokens < Tk and num_patch_tokens % KBLK != 0
    force_last = mixed and not cfg.official_mask
    count = base = None
    if cdf_threshold is not None:
        count, base = ops.cdf_counts(pooled_score, cdf_threshold, min_count=t or 0, force_last=force_last,
                                     want_base=cfg.mode == "vasc")
    if cfg.mode == "vasc":
        if num_patch_tokens is None:
            raise ValueError("CoSA pair debt requires patch metadata")
        if routing_state is None:
            raise ValueError("CoSA pair debt requires routing_state")
        B, H = pooled_score.shape[:2]
        P = (orig_kblk + 1) // 2
        if innovation is None:
            if value is None:
                raise ValueError("CoSA pair debt requires the values or their pair innovation")
            _, _, _, innovation = ops.pool_qkv(v=value[..., :num_patch_tokens, :])
        if base is not None:
            # no hint with a cdf threshold: M is the largest row capacity (SW:3709-3712)
            hint = int(base.max())
        else:
            hint = (t + int(force_last)) if (sparse_ratio is not None and topk is None) else None
            if hint is None:
                hint = max(t, 1) + int(force_last)
        debt, pending, service = _ledger_inputs(routing_state, B, H, P)
        want_stats = routing_stats_store is not None
        sel = ops.select_blocks(pooled_score, mode=_lib.MODE_VASC, topk=t or 0, innovation=innovation,
                                row_cap=base, force_last=force_last, max_capacity=hint, sink_blocks=sink, debt=debt,
                                pending_arrival=pending, prev_service=service,
                                want_priority=True, want_mask=want_stats)
        M = min(hint, orig_kblk)
        _ledger_outputs(routing_state, sel, pooled_score, layer_idx, M, cfg.service_domain, priority, sink)
        if want_stats:
            # the base map the reference hands its selector: Top-K (or the
            # cdf counts) plus the forced mixed tail (SW:7599-7662, 7750-7762)
            if count is not None:
                bm = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=0, row_cap=count,
                                       force_last=force_last, want_mask=True)
            else:
                bm = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=t, force_last=force_last,
                                       want_mask=True)
            base_mask = bm["mask"].bool()
            protected = None
            if force_last:
                protected = torch.zeros_like(base_mask)
                protected[..., orig_kblk - 1] = True
            routing_stats_store.update(_routing_stats(pooled_score, sel, base_mask.sum(-1, dtype=torch.int32),
                                                      base_mask, (debt, pending, service), innovation, protected, M))
    elif count is not None:
        sel = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=0, row_cap=count, force_last=force_last,
                                sink_blocks=sink)
    else:
        sel = ops.select_blocks(pooled_score, mode=_lib.MODE_TOPK, topk=t, force_last=force_last,
                                sink_blocks=sink)
    if routing_stats_store is not None:
        # the layer's resolved PV threshold, 1e10 where it is inactive (SW:7012-7020, 7797-7800)
        thr = resolve_pv_threshold(cfg.pv_threshold, Tk)
        if not pv_threshold_active(cfg.pv_active_layers, layer_idx):
            thr = 1e10
        routing_stats_store["qk_pv_threshold"] = torch.tensor(thr, device=pooled_score.device)
    return sel, total_kblk


def _sparsity(sel: dict, total_kblk: int) -> torch.Tensor:
    """``1 - mean(final_map)`` over the patch and sink columns (SW:8218-8245)."""
    kept = sel["count"].sum(dtype=torch.float64)
    return (1.0 - kept / float(sel["count"].numel() * total_kblk)).float()


def block_sparse_attn_cuda(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                           pooled_score: torch.Tensor, topk: int | None = None, sparse_ratio: float | None = None,
                           cdf_threshold: float | None = None, return_sparsity: bool = False,
                           dtype: torch.dtype = torch.float16, *, layer_idx: int = 0,
                           routing_stats_store: dict | None = None, routing_state: dict | None = None,
                           num_patch_tokens: int | None = None, **research):
    """Sparse global attention of the patch queries (SW:6868-8245).

    query ``[B,H,Nq,D]`` (patch queries), key/value ``[B,H,Tk,D]`` with the
    special tokens appended, pooled_score ``[B,H,ceil(Nq/128),ceil(Np/64)]``.
    The selection mode follows the reference's ``SPARSE_VGGT_*`` switches
    (``vasc`` when ``COSA_VALUE_RISK_PAIR_DEBT`` is on, else ``topk``).
    ``dtype`` is accepted for signature compatibility: the kernel computes
    in bf16. Returns ``o`` (query dtype) or ``(o, sparsity)``.
    """
    _require_gpu(query, "query")
    sel, total_kblk = _select_for_layer(key, value, pooled_score, topk, sparse_ratio, cdf_threshold, layer_idx,
                                        routing_stats_store, routing_state, num_patch_tokens, research)
    vt = ops.pack_v(value)
    thr = _pv_threshold(key, layer_idx)
    if thr is None:
        o = ops.block_sparse_attn(query, key, vt, sel["index"], sel["count"])
        _record_pv_execution(routing_state)
    else:
        o, pv_map = ops.block_sparse_attn_pv(query, key, vt, sel["index"], sel["count"], thr)
        _record_pv_execution(routing_state, pv_map, pooled_score.shape[-1])
    if o.dtype != query.dtype:
        o = o.to(query.dtype)
    if return_sparsity:
        return o, _sparsity(sel, total_kblk)
    return o


def sparse_global_attention(q_patch: torch.Tensor, q_special: torch.Tensor | None, key: torch.Tensor,
                            value: torch.Tensor, pooled_score: torch.Tensor, *, sparse_ratio: float | None = None,
                            topk: int | None = None, cdf_threshold: float | None = None, layer_idx: int = 0,
                            routing_stats_store: dict | None = None, routing_state: dict | None = None,
                            num_patch_tokens: int | None = None, want_sparsity: bool = True,
                            _innovation: torch.Tensor | None = None, token_layout: tuple | None = None,
                            _vt: torch.Tensor | None = None, _priority: torch.Tensor | None = None,
                            **research):
    """``block_sparse_attn_cuda`` for a whole global layer: the selection of
    the patch queries as there, and the special-token queries (which the
    reference runs through a dense SDPA, ATT:8464-8484) over every key in
    the same attention launch. Returns ``(o_patch, o_special, sparsity)``
    in bf16 (``o_special`` None without special queries; ``sparsity`` None
    unless ``want_sparsity``; ``_innovation``: the patch values' pair
    innovation when the caller pooled them with Q and K). With
    ``token_layout = (N, P, S)`` the first result is instead the layer's
    frame-major ``[B, N*P, H*D]`` output (restore included) and the second
    None. ``_vt``: the values already packed as ``ops.pack_v(value)`` (then
    ``value`` may be None); ``_priority``: ``pooled_score`` cleaned as the
    ledger stores it (``ops.pooled_softmax(..., priority=True)``)."""
    _require_gpu(q_patch, "query")
    if value is None and _vt is None:
        raise ValueError("sparse_global_attention requires the values (or their packed tiles)")
    sel, total_kblk = _select_for_layer(key, value, pooled_score, topk, sparse_ratio, cdf_threshold, layer_idx,
                                        routing_stats_store, routing_state, num_patch_tokens, research,
                                        innovation=_innovation, priority=_priority)
    vt = ops.pack_v(value) if _vt is None else _vt
    thr = _pv_threshold(key, layer_idx)
    if thr is None:
        if token_layout is not None:
            out = ops.global_attn_tokens(q_patch, q_special, key, vt, sel["index"], sel["count"], *token_layout)
            _record_pv_execution(routing_state)
            return out, None, (_sparsity(sel, total_kblk) if want_sparsity else None)
        o_patch, o_special = ops.global_attn(q_patch, q_special, key, vt, sel["index"], sel["count"])
        _record_pv_execution(routing_state)
    else:  # the post-cut applies to the patch queries; the special queries stay dense
        o_patch, pv_map = ops.block_sparse_attn_pv(q_patch, key, vt, sel["index"], sel["count"], thr)
        o_special = None if q_special is None else ops.dense_attn(q_special, key, vt)
        _record_pv_execution(routing_state, pv_map, pooled_score.shape[-1])
    if token_layout is not None:
        return ops.restore_tokens(o_patch, o_special, *token_layout), None, \
            (_sparsity(sel, total_kblk) if want_sparsity else None)
    return o_patch, o_special, (_sparsity(sel, total_kblk) if want_sparsity else None)
