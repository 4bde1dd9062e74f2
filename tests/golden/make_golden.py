"""Write golden vectors from the reference's own selector and predictor.

Runs in the build container only (the reference is not present on the GPU
box). The pure-torch functions are loaded from the reference's source text
by AST extraction, as the reference's ``tests/check_selector.py:12-25``
does, and run on the CPU; only their inputs and outputs are saved:

* ``selector_check.npz``  the check_selector protocol (seed 20260906,
  K in {1,2,7,8,31} x protect_last in {F,T} x 24 layers of one
  routing_state) with the release vasc switches;
* ``selector_c1.npz``     a C1-shaped chain (H=2, 65 query blocks x 130 key
  blocks, budget int(130*0.25)=32 + protected mixed tail) over 6 layers of
  unit-temperature scores, where the ledger accrues debt and the gate both
  opens and closes;
* ``predict.npz``         ``predict_attention`` on bf16 inputs under CPU bf16
  autocast (ragged token counts);
* ``selector_scale.npz``  the at-scale chains of ``scale_cases.py`` (C1 with
  all 16 heads over 6 layers, the C2 block shape over 3 layers): only the
  reference's outputs (bit-packed selections and the ledger per layer) and a
  digest of the inputs, which the test regenerates.

Usage: ``python tests/golden/make_golden.py [/root/reference]``.
"""
from __future__ import annotations

import ast
import math
import os
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent
SELECTOR_FUNCS = {"_project_conservative_capped_mass", "_reduce_pv_service_to_pair",
                  "_reduce_qk_admission_to_pair", "_reduce_qk_indices_to_pair",
                  "get_cosa_value_risk_pair_debt_mask", "finalize_cosa_value_risk_pair_debt"}
RELEASE_SWITCHES = dict(FUSED_ROUTING="0", CONSERVATIVE_ARRIVAL_PROJECTION="1", CONSERVATIVE_DEBT_PROJECTION="1",
                        INPLACE_ARRIVAL_PROJECTION="0", UNIFORM_CAPACITY_HINT="0", COUNTERFACTUAL_STATS="0",
                        SERVICE_LEDGER_OBSERVER="0", POSTCUT_ORDER_OBSERVER="0", DEBT_SERVICE_DOMAIN="qk_admission",
                        INDEX_SERVICE_REDUCTION="1", SORT_SELECTED_INDICES="1")


def extract(path: Path, names: set, namespace: dict) -> dict:
    tree = ast.parse(path.read_text(encoding="utf-8"))
    nodes = [n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name in names]
    assert {n.name for n in nodes} == names, f"missing {names - {n.name for n in nodes}}"
    future = ast.ImportFrom(module="__future__", names=[ast.alias(name="annotations")], level=0)
    module = ast.fix_missing_locations(ast.Module(body=[future, *nodes], type_ignores=[]))
    exec(compile(module, str(path), "exec"), namespace)
    return namespace


def _np(t):
    return t.detach().cpu().numpy()


def selector_chain(fn, rng_torch, K, Q, H, layers, protect_last, *, capacity_fn, hint=None, peak=1.0,
                   stats=False):
    """Run one routing_state chain; return per-layer arrays (with ``stats``
    also the selector's routing statistics per layer, ``stat_<key>``)."""
    state = {}
    rec = {k: [] for k in ("score", "value", "cap", "protected", "selected", "priority", "debt", "arrival",
                           "service", "indices")}
    stat_rec: dict = {}
    for layer in range(layers):
        scores = (torch.randn(1, H, Q, K, generator=rng_torch) * peak).softmax(-1)
        values = torch.randn(1, H, K, 13, generator=rng_torch)
        capacity = capacity_fn(scores)
        base = torch.arange(K).view(1, 1, 1, -1) < capacity
        protected = torch.zeros_like(base)
        if protect_last:
            protected[..., -1:] = capacity > 0
        store = {} if stats else None
        selected = fn(scores, values, base, layer_idx=layer, routing_state=state, protected_mask=protected,
                      fp32_projection=True, max_capacity_hint=hint, stats_store=store)
        for key, val in (store or {}).items():
            stat_rec.setdefault(f"stat_{key}", []).append(_np(val))
        rec["score"].append(_np(scores))
        rec["value"].append(_np(values))
        rec["cap"].append(_np(capacity[..., 0]))
        rec["protected"].append(_np(protected))
        rec["selected"].append(_np(selected))
        rec["priority"].append(_np(state["cosa_value_risk_pair_priority"]))
        rec["debt"].append(_np(state["cosa_value_risk_pair_debt"]))
        rec["arrival"].append(_np(state["cosa_value_risk_pair_pending_arrival"]))
        rec["service"].append(_np(state["qk_pv_service_observation"]["pair_service_fraction"]))
        idx = _np(state["cosa_value_risk_pair_selected_indices"])
        rec["indices"].append(idx)
    out = {k: np.stack(v) for k, v in rec.items() if k != "indices"}
    out.update({k: np.stack(v) for k, v in stat_rec.items()})
    return out, state


def main(ref_root: Path) -> None:
    torch.set_num_threads(2)
    for key in list(os.environ):
        if key.startswith("SPARSE_VGGT_"):
            del os.environ[key]
    os.environ.update({"SPARSE_VGGT_COSA_" + k: v for k, v in RELEASE_SWITCHES.items()})
    sw = ref_root / "src/sparse_vggt/utils/sparse_wrapper.py"
    ns = extract(sw, SELECTOR_FUNCS, dict(torch=torch, F=F, os=os))
    fn, fin = ns["get_cosa_value_risk_pair_debt_mask"], ns["finalize_cosa_value_risk_pair_debt"]

    # 1. check_selector protocol
    torch.manual_seed(20260906)
    gen = torch.default_generator
    arrays = {}
    for K in (1, 2, 7, 8, 31):
        for protect in (False, True):
            rec, state = selector_chain(fn, gen, K, 3, 2, 24, protect,
                                        capacity_fn=lambda s: torch.randint(s.shape[-1] + 1, (1, 2, 3, 1)))
            terminal = fin(state)
            rec["terminal_debt"] = _np(state["cosa_value_risk_pair_debt"])
            rec["terminal_nonempty"] = np.array(bool(terminal))
            rec["second_finalize_empty"] = np.array(fin(state) == {})
            for k, v in rec.items():
                arrays[f"K{K}_p{int(protect)}_{k}"] = v
    np.savez_compressed(OUT / "selector_check.npz", **arrays)

    # 2. C1-shaped chain with the block_sparse_attn_cuda capacity rule
    gen = torch.Generator().manual_seed(1)
    K, Q, H = 130, 65, 2
    topk = int(K * (1 - 0.75))

    def c1_capacity(scores):
        top = torch.topk(scores, topk, dim=-1).indices
        base = torch.zeros_like(scores, dtype=torch.bool).scatter_(-1, top, True)
        base[..., K - 1] = True
        return base.sum(-1, keepdim=True)

    # routing statistics with the reference's default counterfactual statistics on
    os.environ["SPARSE_VGGT_COSA_COUNTERFACTUAL_STATS"] = "1"
    rec, state = selector_chain(fn, gen, K, Q, H, 6, True, capacity_fn=c1_capacity, hint=topk + 1, peak=1.0,
                                stats=True)
    os.environ["SPARSE_VGGT_COSA_COUNTERFACTUAL_STATS"] = RELEASE_SWITCHES["COUNTERFACTUAL_STATS"]
    terminal = {}
    fin(state, stats_store=terminal)
    rec["terminal_debt"] = _np(state["cosa_value_risk_pair_debt"])
    for key, val in terminal.items():
        rec[f"terminal_stat_{key}"] = _np(val)
    np.savez_compressed(OUT / "selector_c1.npz", **rec)

    # 3. predict_attention under CPU bf16 autocast
    att = ref_root / "src/sparse_vggt/models/attention.py"
    from einops import rearrange
    ns2 = extract(att, {"predict_attention"}, dict(torch=torch, F=F, math=math, rearrange=rearrange, os=os))
    pa = ns2["predict_attention"]
    out = {}
    g = torch.Generator().manual_seed(7)
    for i, (nq, nk) in enumerate(((300, 300), (1000, 1041), (128, 64))):
        q = (torch.randn(1, 2, nq, 64, generator=g) * 2).to(torch.bfloat16)
        k = (torch.randn(1, 2, nk, 64, generator=g) * 2).to(torch.bfloat16)
        with torch.autocast("cpu", dtype=torch.bfloat16):
            prob = pa(q, k)
            _, var = pa(q, k, return_key_block_variance=True)
            _, var_max = pa(q, k, pool_mode="max", return_key_block_variance=True)
        out[f"var{i}"] = var.float().numpy()
        out[f"var_max{i}"] = var_max.float().numpy()
        out[f"q{i}"] = q.float().numpy()
        out[f"k{i}"] = k.float().numpy()
        out[f"prob{i}"] = prob.float().numpy()
        out[f"prob_dtype{i}"] = np.array(str(prob.dtype))
    np.savez_compressed(OUT / "predict.npz", **out)

    # 4. at-scale chains (inputs regenerated by the test from scale_cases.py)
    sys.path.insert(0, str(OUT))
    import scale_cases
    scale = {}
    for case in scale_cases.CASES:
        state = {}
        hashes = []
        for layer, scores, values, capacity, protected, hint in scale_cases.layer_inputs(case):
            selected = fn(scores, values, torch.arange(scores.shape[-1]).view(1, 1, 1, -1) < capacity,
                          layer_idx=layer, routing_state=state, protected_mask=protected, fp32_projection=True,
                          max_capacity_hint=hint)
            hashes.append(scale_cases.digest(_np(scores), _np(values), _np(capacity), _np(protected)))
            scale[f"{case}_l{layer}_selected"] = np.packbits(_np(selected).astype(bool), axis=-1)
            scale[f"{case}_l{layer}_debt"] = _np(state["cosa_value_risk_pair_debt"])
            scale[f"{case}_l{layer}_arrival"] = _np(state["cosa_value_risk_pair_pending_arrival"])
            scale[f"{case}_l{layer}_service"] = _np(state["qk_pv_service_observation"]["pair_service_fraction"])
        scale[f"{case}_digest"] = np.array(scale_cases.digest(np.array(hashes)))
    np.savez_compressed(OUT / "selector_scale.npz", **scale)
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
