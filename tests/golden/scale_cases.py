"""Inputs of the at-scale selector chains, regenerated bit-identically by
``make_golden.py`` (which runs the reference's selector on them) and by
``tests/test_golden.py`` (which replays them through the oracle), so the
fixture holds only the reference's outputs.

Each case is one routing_state chain of layers of the release vasc selector
(``get_cosa_value_risk_pair_debt_mask``, ``sparse_wrapper.py:3632-4098``):

* ``c1_full``: config 1's block shape with all 16 heads: 65 query blocks x
  130 key blocks, budget int(130 * 0.25) = 32 plus the protected mixed tail
  block (the hint is 33), 6 layers;
* ``c2``: config 2's block shape: 16 heads, 259 x 518 blocks, the
  structural profile's capacities (120 and 155 per row, hint = capacity),
  no protected tail (VGGT's official mask), 3 layers. A per-head column
  bias shared by every row concentrates the demand, so unserved arrival
  accrues debt in the ledger from layer 1 on.

Scores are row softmaxes of scaled Gaussian logits (plus the column bias),
pooled values are Gaussian [B, H, K, 64]; everything comes from one seeded
CPU ``torch.Generator`` per case, drawn in a fixed order.
"""
from __future__ import annotations

import hashlib

import numpy as np
import torch

CASES = {
    "c1_full": dict(K=130, Q=65, H=16, layers=6, caps=[32] * 6, protect_last=True, peak=1.0, bias=0.0, seed=11),
    "c2": dict(K=518, Q=259, H=16, layers=3, caps=[120, 155, 120], protect_last=False, peak=1.0, bias=3.0,
               seed=12),
}


def layer_inputs(case: str):
    """Yield ``(layer, scores [1,H,Q,K] f32, values [1,H,K,64] f32, capacity
    [1,H,Q,1] int64, protected [1,H,Q,K] bool, hint)`` for every layer."""
    c = CASES[case]
    K, Q, H = c["K"], c["Q"], c["H"]
    gen = torch.Generator().manual_seed(c["seed"])
    bias = torch.randn(1, H, 1, K, generator=gen) * c["bias"]
    for layer in range(c["layers"]):
        scores = (torch.randn(1, H, Q, K, generator=gen) * c["peak"] + bias).softmax(-1)
        values = torch.randn(1, H, K, 64, generator=gen)
        t = c["caps"][layer]
        # block_sparse_attn_cuda's capacity: the Top-K base map plus the
        # forced mixed tail when it is protected (SW:7599-7662, 7744-7750)
        top = torch.topk(scores, t, dim=-1).indices
        base = torch.zeros_like(scores, dtype=torch.bool).scatter_(-1, top, True)
        protected = torch.zeros_like(base)
        if c["protect_last"]:
            base[..., K - 1] = True
            protected[..., K - 1] = True
        capacity = base.sum(-1, keepdim=True)
        hint = t + int(c["protect_last"])
        yield layer, scores, values, capacity, protected, hint


def digest(*arrays) -> str:
    """sha256 of the arrays' bytes: the test checks it to know that its
    regenerated inputs are the ones the fixture was made from."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(np.asarray(a)).tobytes())
    return h.hexdigest()
