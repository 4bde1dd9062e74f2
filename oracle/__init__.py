"""CPU oracle for the VASC sparse global-attention path.

TEST INFRASTRUCTURE ONLY. Nothing under ``vasc_amd/`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker of the HIP path.

Modules
-------
canon      canonical fp32/fp64 reductions shared bit-for-bit with the HIP
           select kernels (wave-tree and sequential fp64 sums).
pooling    block mean pooling (``avg_pool1d(ceil_mode=True)`` semantics) and
           the pooled-score softmax of ``predict_attention``.
selector   Top-K block mask, the VASC value-risk pair-debt selector with its
           cross-layer ledger, terminal settlement and the QK-admission
           service reduction.
lut        the delta-encoded LUT of SpargeAttn and ascending index lists.
attention  masked (block-sparse) softmax attention in float64.
profile    the structural layer-budget profile and per-layer capacities.

Parity status of each function is stated in its module header.
"""
