"""Installers of the sparse global attention into VGGT/Pi3-shaped models.

Mirrors the reference's model adapters:

* ``sparse_aggregator_from_vggt`` (``src/sparse_vggt/models/vggt.py:215-299``)
  and ``sparse_aggregator_from_vggt_layerwise``
  (``src/sparse_vggt/models/vggt_layerwise.py:21-1746``, the per-layer ratio
  path of the release launcher, 1099-1101, 1237, 1271-1278);
* ``sparse_model_from_pi3`` (``src/sparse_vggt/models/pi3.py:138-233``): the
  odd decoder layers are global, logical layer ``i // 2``.

Each patches the global blocks' ``attn.forward`` with
``adaptive_sparse_attention_forward`` bound to the layer's sparsity, hangs
one ``routing_state`` dict (the cross-layer ledger) on the model and on
every patched attention module, and returns ``(model, aux_output_store)``.
The models clear the ledger at the start of each forward and settle it
after the last layer (``vasc_amd.aggregator``). Research options of the
reference (Hilbert order, the ~20 layer-wise routing modes) are rejected
when enabled.
"""
from __future__ import annotations

from functools import partial
from types import MethodType

from .attention import adaptive_sparse_attention_forward
from .sparse_wrapper import check_sparse_mode


def _reject(**flags) -> None:
    for name, value in flags.items():
        if value:
            raise NotImplementedError(f"{name} selects a research path that this build does not implement")


def _install(attn_modules, layer_ratios, *, cdf_threshold, pool_mode, aux_output, aux_sparsity_only,
             num_special_tokens, routing_state):
    aux_output_store = {i: ({} if aux_output else None) for i in range(len(attn_modules))}
    for i, attn in enumerate(attn_modules):
        fwd = partial(adaptive_sparse_attention_forward, sparse_ratio=layer_ratios[i], cdf_threshold=cdf_threshold,
                      pool_mode=pool_mode, aux_output_store=aux_output_store[i],
                      aux_sparsity_only=aux_sparsity_only, num_special_tokens=num_special_tokens,
                      num_heads=attn.num_heads, layer_idx=i, routing_state=routing_state)
        attn.forward = MethodType(fwd, attn)
        attn._sparse_routing_state = routing_state
    return aux_output_store


def sparse_aggregator_from_vggt(aggregator, use_hilbert: bool = False, sparse_ratio: float | None = None,
                                cdf_threshold: float | None = None, pool_mode: str = "avg", aux_output: bool = False,
                                aux_sparsity_only: bool = True, num_special_tokens: int = 5,
                                analyze_importance_blocks: bool = False, analyze_block_selection: bool = False,
                                verbose: bool = True):
    """Uniform sparsity on all global blocks (vggt.py:215-299)."""
    check_sparse_mode(sparse_ratio, cdf_threshold)
    _reject(use_hilbert=use_hilbert, analyze_importance_blocks=analyze_importance_blocks,
            analyze_block_selection=analyze_block_selection)
    n = len(aggregator.global_blocks)
    return sparse_aggregator_from_vggt_layerwise(aggregator, layer_sparsity_ratios=[sparse_ratio] * n,
                                                 cdf_threshold=cdf_threshold, pool_mode=pool_mode,
                                                 aux_output=aux_output, aux_sparsity_only=aux_sparsity_only,
                                                 num_special_tokens=num_special_tokens, verbose=verbose)


def sparse_aggregator_from_vggt_layerwise(aggregator, use_hilbert: bool = False, layer_config: dict | None = None,
                                          layer_sparsity_ratios: list[float] | None = None,
                                          sparse_ratio: float | None = None, cdf_threshold: float | None = None,
                                          pool_mode: str = "avg", aux_output: bool = False,
                                          aux_sparsity_only: bool = True, num_special_tokens: int = 5,
                                          verbose: bool = True, **research):
    """Per-layer sparsity from ``layer_sparsity_ratios`` (one per global block)
    or ``layer_config {i: {"sparse_ratio": r}}``; falls back to the uniform
    ``sparse_ratio`` (vggt_layerwise.py:1099-1101, 1237, 1271-1278)."""
    _reject(use_hilbert=use_hilbert, **{k: v for k, v in research.items() if k.startswith("use_")})
    n = len(aggregator.global_blocks)
    if layer_sparsity_ratios is not None:
        ratios = [float(r) for r in layer_sparsity_ratios]
    elif layer_config is not None:
        ratios = [float(layer_config.get(i, {}).get("sparse_ratio", sparse_ratio)) for i in range(n)]
    else:
        ratios = [sparse_ratio] * n
    if len(ratios) != n:
        raise ValueError(f"layer_sparsity_ratios must hold {n} values")
    for r in ratios:
        check_sparse_mode(r, cdf_threshold)
        if r is not None and not 0.0 <= r <= 1.0:
            raise ValueError("layer sparsity ratios must be in [0, 1]")
    routing_state: dict = {}
    aggregator._sparse_routing_state = routing_state
    store = _install([blk.attn for blk in aggregator.global_blocks], ratios, cdf_threshold=cdf_threshold,
                     pool_mode=pool_mode, aux_output=aux_output, aux_sparsity_only=aux_sparsity_only,
                     num_special_tokens=num_special_tokens, routing_state=routing_state)
    aggregator._sparse_aux_output_store = store
    if verbose:
        print(f"sparse global attention on {n} layers: sparsity {ratios}")
    return aggregator, store


def sparse_model_from_pi3(model, use_hilbert: bool = False, sparse_ratio: float | None = None,
                          layer_sparsity_ratios: list[float] | None = None, cdf_threshold: float | None = None,
                          pool_mode: str = "avg", aux_output: bool = False, aux_sparsity_only: bool = True,
                          num_special_tokens: int = 5, verbose: bool = True):
    """Sparse global attention on the odd decoder layers of a Pi3-shaped
    model (pi3.py:138-233); logical layer ``i // 2``."""
    check_sparse_mode(sparse_ratio, cdf_threshold)
    _reject(use_hilbert=use_hilbert)
    global_layers = [i for i in range(len(model.decoder)) if i % 2 == 1]
    n = len(global_layers)
    if layer_sparsity_ratios is not None:
        if len(layer_sparsity_ratios) != n:
            raise ValueError(f"Pi3 layer_sparsity_ratios must match the {n} global-attention layers")
        if any(r < 0.0 or r > 1.0 for r in layer_sparsity_ratios):
            raise ValueError("Pi3 layer sparsity ratios must be in [0, 1]")
        ratios = [float(r) for r in layer_sparsity_ratios]
    else:
        ratios = [sparse_ratio] * n
    routing_state: dict = {}
    model._sparse_routing_state = routing_state
    store = _install([model.decoder[i].attn for i in global_layers], ratios, cdf_threshold=cdf_threshold,
                     pool_mode=pool_mode, aux_output=aux_output, aux_sparsity_only=aux_sparsity_only,
                     num_special_tokens=num_special_tokens, routing_state=routing_state)
    model._sparse_aux_output_store = store
    if verbose:
        print(f"Pi3 global layer sparsity: {ratios}")
    return model, store


def install_for_mode(model, backbone: str, mode: str, sparsity: float, structural_allocation: bool | None = None,
                     **kwargs):
    """Mode, sparsity and structural allocation as explicit arguments, as
    the reference's evaluators apply them (evaluate.py:35-52, 183-231): the
    per-layer ratios of ``allocation_settings`` installed with the backbone's
    layer-wise installer; ``dense`` leaves the model as it is (the unpatched
    upstream model). The kernels read the mode's switches at call time, so
    run the model inside ``launcher.use_mode(backbone, mode)``. Returns
    ``(model, aux_output_store or None, settings)``."""
    from .launcher import MODES, allocation_settings
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}")
    settings = allocation_settings(backbone, mode, sparsity, structural_allocation)
    if mode == "dense":
        return model, None, settings
    ratios = settings["layer_sparsities"]
    if backbone == "vggt":
        model, store = sparse_aggregator_from_vggt_layerwise(model, layer_sparsity_ratios=ratios, **kwargs)
    elif backbone == "pi3":
        model, store = sparse_model_from_pi3(model, sparse_ratio=sparsity, layer_sparsity_ratios=ratios, **kwargs)
    else:
        raise ValueError("backbone must be vggt or pi3")
    return model, store, settings
