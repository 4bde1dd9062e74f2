"""Mode switch and structural layer-budget profile of the VASC launcher.

Mirrors ``evaluate.py:12-80`` of the reference: the paper constants
(``vasc_amd/configs/paper.json``, the reference's ``configs/paper.json``), ``layer_sparsity`` (favoured layers get ``s-delta``,
the others ``s + n_fav*delta/(L-n_fav)``, only above ``enable_above``),
``allocation_settings`` and ``method_environment`` (the ``SPARSE_VGGT_*``
switches of the three release modes). ``routing_config`` resolves those
switches into the explicit settings the GPU path uses, so launches that set
the reference's environment keep working.
"""
from __future__ import annotations

import json
import math
import os
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path

MODES = ("dense", "topk", "vasc")

# The paper constants (the reference's configs/paper.json): evaluation stride,
# the sparsity sweep and the structural layer-budget profile.
CONFIG = json.loads((Path(__file__).resolve().parent / "configs" / "paper.json").read_text(encoding="utf-8"))


def layer_sparsity_string(backbone: str, sparsity: float, allocation: str):
    """The ``%.10f``-joined profile string, or None (evaluate.py:16-32)."""
    if backbone not in ("vggt", "pi3") or allocation not in ("paper", "uniform"):
        raise ValueError("unsupported backbone or allocation")
    if not 0 <= sparsity < 1:
        raise ValueError("sparsity must be in [0, 1)")
    policy = CONFIG["structural"]
    if allocation == "uniform" or sparsity <= policy["enable_above"]:
        return None
    shape = policy[backbone]
    selected = shape["favored_layers_zero_based"]
    delta = policy["delta"]
    offset = len(selected) * delta / (shape["layers"] - len(selected))
    values = [sparsity - delta if i in selected else sparsity + offset for i in range(shape["layers"])]
    if any(not 0 <= x < 1 for x in values):
        raise ValueError("structural profile leaves [0, 1); use uniform allocation")
    return ",".join(f"{v:.10f}" for v in values)


def layer_sparsity(backbone: str, sparsity: float, allocation: str = "paper"):
    """Per-layer sparsity list as the evaluators parse it back, or None."""
    s = layer_sparsity_string(backbone, sparsity, allocation)
    return None if s is None else [float(x) for x in s.split(",")]


def allocation_settings(backbone: str, mode: str, sparsity: float, structural_allocation: bool | None = None):
    """``allocation_settings`` of evaluate.py:35-52 with explicit arguments."""
    enabled = CONFIG["structural"]["enabled"] if structural_allocation is None else bool(structural_allocation)
    policy = "paper" if enabled and mode != "dense" else "uniform"
    profile = layer_sparsity(backbone, sparsity, policy)
    ratios = profile if profile is not None else (
        [0.0 if mode == "dense" else sparsity] * CONFIG["structural"][backbone]["layers"])
    return {
        "enabled": enabled,
        "applied": profile is not None,
        "effective_policy": "dense" if mode == "dense" else ("paper" if profile is not None else "uniform"),
        "requested_sparsity": sparsity,
        "layer_sparsities": ratios,
    }


def method_environment(backbone: str, mode: str) -> dict:
    """The ``SPARSE_VGGT_*`` switches of a release mode (evaluate.py:55-80)."""
    if backbone not in ("vggt", "pi3") or mode not in MODES:
        raise ValueError("unsupported backbone or mode")
    active = mode == "vasc"
    values = {
        "COSA_VALUE_RISK_PAIR_DEBT": int(active),
        "COSA_PRODUCTION_FAST": 1,
        "COSA_ORDERED_LUT": 0,
        "COSA_TOPK_ORDERED_LUT": 0,
        "COSA_COMPACT_ORDERED_LUT": 0,
        "COSA_HRM_ORDERED_LUT": 0,
        "COSA_FP32_PROJECTION": int(active or backbone == "vggt"),
        "COSA_DEBT_SERVICE_DOMAIN": "qk_admission" if active or backbone == "vggt" else "pv_execution",
        "COSA_KERNEL_PAIR_SERVICE": 0,
        "COSA_INDEX_SERVICE_REDUCTION": int(active),
        "COSA_CONSERVATIVE_DEBT_PROJECTION": int(active),
        "COSA_CONSERVATIVE_ARRIVAL_PROJECTION": int(active),
        "COSA_PV_COUNT_STATS": 0,
        "COLLECT_QK_PV_SERVICE": 0,
        "SKIP_ROUTING_STATS": 1,
        "QK_PV_THRESHOLD": "1e10",
    }
    if backbone == "vggt" and mode != "dense":
        values["OFFICIAL_MASK"] = 1
    return {"SPARSE_VGGT_" + k: str(v) for k, v in values.items()}


@contextmanager
def use_mode(backbone: str, mode: str):
    """The release mode as an explicit argument: inside the block the
    process environment holds exactly the ``SPARSE_VGGT_*`` switches of
    ``method_environment(backbone, mode)`` (the reference's evaluators export
    them for the whole process, evaluate.py:55-80, 193-195); the previous
    switches are restored on exit."""
    env = method_environment(backbone, mode)
    saved = {k: os.environ.pop(k) for k in list(os.environ) if k.startswith("SPARSE_VGGT_")}
    os.environ.update(env)
    try:
        yield env
    finally:
        for k in [k for k in os.environ if k.startswith("SPARSE_VGGT_")]:
            del os.environ[k]
        os.environ.update(saved)


_TRUE = {"1", "true", "yes", "on"}


def _flag(env, name: str, default: str = "0") -> bool:
    return env.get("SPARSE_VGGT_" + name, default).lower() in _TRUE


@dataclass(frozen=True)
class RoutingConfig:
    """Explicit selection settings of the sparse op."""
    mode: str = "vasc"          # "topk" or "vasc" (dense never reaches the op)
    official_mask: bool = False  # VGGT: no forced/protected mixed-tail block
    skip_routing_stats: bool = True
    service_domain: str = "qk_admission"  # ledger service: "qk_admission" or "pv_execution"
    pv_threshold: str = "1e10"   # SPARSE_VGGT_QK_PV_THRESHOLD (resolved per layer)
    pv_active_layers: str = ""   # SPARSE_VGGT_QK_PV_ACTIVE_LAYERS (empty: every layer)


def routing_config(env=None) -> RoutingConfig:
    """Resolve the reference's environment switches into a RoutingConfig.

    Only the release combinations are accepted; research switches that
    change the algorithm raise ``NotImplementedError`` instead of being
    silently ignored.
    """
    env = os.environ if env is None else env
    vasc = _flag(env, "COSA_VALUE_RISK_PAIR_DEBT")
    unsupported = [n for n in ("COSA_ORDERED_LUT", "COSA_TOPK_ORDERED_LUT", "COSA_COMPACT_ORDERED_LUT",
                               "COSA_HRM_ORDERED_LUT", "COSA_KERNEL_PAIR_SERVICE", "PROJECTED_QK_DEBT",
                               "PROJECTED_QK_PV_DEBT", "COSA_BUDGET_ONLY_UPSTREAM", "COSA_UNIFORM_CAPACITY_HINT",
                               "COSA_RISK_SAFE_OBSERVER", "QK_VALUE_RISK_OBSERVER", "QK_BUNDLE_OBSERVER",
                               "COLLECT_QK_PV_SERVICE", "RADIAL_A_DENSE", "RADIAL_A_CHUNKED")
                   if _flag(env, n)]
    domain = "qk_admission"
    if vasc:
        domain = env.get("SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN", "pv_execution").lower()
        if domain not in ("qk_admission", "pv_execution"):
            raise ValueError("unsupported CoSA debt service domain")
        if not _flag(env, "COSA_CONSERVATIVE_ARRIVAL_PROJECTION"):
            unsupported.append("COSA_CONSERVATIVE_ARRIVAL_PROJECTION=0")
        if not _flag(env, "COSA_CONSERVATIVE_DEBT_PROJECTION"):
            unsupported.append("COSA_CONSERVATIVE_DEBT_PROJECTION=0")
    threshold = env.get("SPARSE_VGGT_QK_PV_THRESHOLD", "1e10")
    if threshold != "sequence_mass_bound":
        try:
            resolve_pv_threshold(threshold, 2)
        except ValueError as exc:
            raise ValueError(str(exc)) from None
    if unsupported:
        raise NotImplementedError("switches outside the release modes: " + ", ".join(unsupported))
    return RoutingConfig(mode="vasc" if vasc else "topk", official_mask=_flag(env, "OFFICIAL_MASK"),
                         skip_routing_stats=_flag(env, "SKIP_ROUTING_STATS"), service_domain=domain,
                         pv_threshold=threshold, pv_active_layers=env.get("SPARSE_VGGT_QK_PV_ACTIVE_LAYERS", ""))


def resolve_pv_threshold(spec: str, key_tokens: int) -> float:
    """The PV post-cut threshold in log2 score units (SW:3064-3087):
    ``sequence_mass_bound`` -> ln(max(N, 2)); ``natural_gap:x`` -> x * log2 e;
    otherwise a non-negative number."""
    if key_tokens <= 0:
        raise ValueError("key token count must be positive")
    if spec == "sequence_mass_bound":
        return math.log(float(max(key_tokens, 2)))
    if spec.startswith("natural_gap:"):
        gap = float(spec.split(":", 1)[1])
        if not math.isfinite(gap) or gap < 0.0:
            raise ValueError("natural-logit PV gap must be finite and non-negative")
        return gap * math.log2(math.e)
    value = float(spec)
    if not math.isfinite(value) or value < 0.0:
        raise ValueError("SPARSE_VGGT_QK_PV_THRESHOLD must be non-negative or sequence_mass_bound")
    return value


def pv_threshold_active(spec: str, layer_idx: int) -> bool:
    """Whether the PV post-cut runs at this global layer (SW:3090-3101):
    every layer when ``spec`` is empty, else the listed layer indices."""
    spec = spec.strip()
    if not spec:
        return True
    return layer_idx in {int(t.strip()) for t in spec.split(",") if t.strip()}
