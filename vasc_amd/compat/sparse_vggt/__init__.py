"""Import shim: the reference package's module names, served by ``vasc_amd``.

The reference's dataset evaluators import ``sparse_vggt``
(``evaluation/eval_7scenes_sparse_vggt.py:939-941, 1115-1118``,
``evaluation/eval_pi3_sparse.py:203``). The run launcher puts this shim's
parent directory on the evaluator's ``PYTHONPATH`` ahead of everything else,
so those imports resolve to this build's modules:

* ``sparse_vggt.utils.sparse_wrapper``   -> ``vasc_amd.sparse_wrapper``
* ``sparse_vggt.models.attention``       -> ``vasc_amd.attention``
* ``sparse_vggt.models.vggt``, ``.vggt_layerwise``, ``.pi3`` -> ``vasc_amd.install``

Each shim module replaces itself in ``sys.modules`` with the ``vasc_amd``
module, so ``module.__file__`` (which the evaluators record as provenance)
names the file that actually runs. ``sparse_vggt.evaluation`` (the Pi3
reconstruction protocol) is not part of this build and fails on import.
"""
__all__ = ["sparse_aggregator_from_vggt", "sparse_model_from_pi3"]


def __getattr__(name):
    if name in __all__:
        from vasc_amd import install
        return getattr(install, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
