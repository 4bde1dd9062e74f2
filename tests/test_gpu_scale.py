"""Attention parity at the benchmark configurations' full sequence lengths.

The float64 oracle (``oracle.attention.block_sparse_attention``) evaluates a
seeded sample of query blocks (always including the first and the last,
partial one) on the same bf16 inputs and the same index lists the kernel
ran; the tolerance is the north star's, max-abs <= 2e-2 and mean-abs <= 2e-3
over the sampled rows. These shapes exercise the kernel's 64-bit head bases
and 32-bit per-block offsets at the sizes the benchmark runs:

* C2: 32 frames x 1041 tokens (33 152 patch queries, 33 312 keys), lists
  from the VASC selector on the C2 synthetic recipe, special-token queries
  in the same launch (dense, every row checked);
* C3: 128 frames (133 248 keys), one head, VASC lists at the structural
  profile's 0.875-sparsity budget;
* C5: 16k and 64k tokens with Poisson block lists (the benchmark's
  ``c5_lists``: forced frame-start columns, variable counts per row).
"""
import math

import numpy as np
import pytest
import torch

import bench
from oracle import attention as OA

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _sample(qb: int, n: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    picks = {0, qb - 1}
    picks.update(int(x) for x in rng.choice(qb, size=min(n, qb), replace=False))
    return sorted(picks)


def _check_sampled(out, q, k, v, index, count, blocks, nq):
    """Compare the kernel output with the oracle on the rows of ``blocks``."""
    idx = index.cpu().numpy()
    cnt = count.cpu().numpy()
    ref = OA.block_sparse_attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                    idx, cnt, q_blocks=blocks)
    rows = np.concatenate([np.arange(i * 128, min((i + 1) * 128, nq)) for i in blocks])
    got = out.float().cpu().numpy()[:, :, rows].astype(np.float64)
    assert np.isfinite(got).all()
    err = np.abs(got - ref[:, :, rows])
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (err.max(), err.mean())
    return err.max(), err.mean()


def _vasc_lists(q, k, v, ratio):
    from vasc_amd import ops, pipeline
    n_patch = q.shape[2]
    plan = pipeline.LayerPlan.make(n_patch, k.shape[2])
    pq, pk, _, iota = ops.pool_qkv(q, k[:, :, :n_patch], v[:, :, :n_patch])
    prob = ops.pooled_softmax(pq, pk)
    sel = pipeline.select_layer(prob, iota, plan, mode="vasc", sparse_ratio=ratio, official_mask=True,
                                ledger=pipeline.Ledger(), layer_idx=0)
    return sel["index"], sel["count"], plan


def test_c2_vasc_lists_with_special_queries():
    from vasc_amd import ops
    from vasc_amd.launcher import layer_sparsity
    dev = torch.device("cuda:0")
    N, P, S, H, D = 32, 1041, 5, 2, 64
    q, k, v = bench.synthetic_layer(N, P, S, H, D, seed=0, device=dev)
    ratio = layer_sparsity("vggt", 0.75, "paper")[0]
    index, count, plan = _vasc_lists(q, k, v, ratio)
    assert plan.q_blocks == 259 and plan.k_blocks == 518 and plan.sink == 3
    c = count.cpu().numpy()
    assert (c == 120 + 3).all(), np.unique(c)  # structural budget 120 plus the 3 sink blocks
    g = torch.Generator(device=dev).manual_seed(7)
    qs = torch.randn(1, H, N * S, D, device=dev, generator=g).to(torch.bfloat16)
    vt = ops.pack_v(v)
    o_p, o_s = ops.global_attn(q, qs, k, vt, index, count)
    torch.cuda.synchronize()
    _check_sampled(o_p, q, k, v, index, count, _sample(plan.q_blocks, 10, 1), q.shape[2])
    dl, dc = OA.dense_lists(1, H, N * S, N * P)
    ref = OA.block_sparse_attention(qs.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                    dl, dc)
    err = np.abs(o_s.float().cpu().numpy() - ref)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (err.max(), err.mean())
    # the same launch without the special queries gives the same patch rows
    alone = ops.block_sparse_attn(q, k, vt, index, count)
    assert torch.equal(alone.view(torch.int16), o_p.view(torch.int16))


def test_c3_vasc_lists_one_head():
    from vasc_amd import ops
    from vasc_amd.launcher import layer_sparsity
    dev = torch.device("cuda:0")
    N, P, S, H, D = 128, 1041, 5, 1, 64
    q, k, v = bench.synthetic_layer(N, P, S, H, D, seed=3, device=dev)
    ratios = layer_sparsity("vggt", 0.875, "paper")
    index, count, plan = _vasc_lists(q, k, v, ratios[0])
    assert plan.k_blocks == 2072 and plan.sink == 10
    assert (count.cpu().numpy() == 224 + 10).all()
    o = ops.block_sparse_attn(q, k, ops.pack_v(v), index, count)
    torch.cuda.synchronize()
    _check_sampled(o, q, k, v, index, count, _sample(plan.q_blocks, 14, 3), q.shape[2])


@pytest.mark.parametrize("T", [16384, 65536])
@pytest.mark.parametrize("rho", [0.1, 0.25, 0.5])
def test_c5_poisson_lists(T, rho):
    from vasc_amd import ops
    dev = torch.device("cuda:0")
    H, D = 2, 64
    g = torch.Generator(device=dev).manual_seed(T + int(rho * 1000))
    q, k, v = (torch.randn(1, H, T, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    index, count = bench.c5_lists(T, H, rho, seed=int(rho * 100) + T, device=dev)
    kb = T // 64
    c = count.cpu().numpy()
    assert c.min() >= 1 and c.max() <= kb
    assert abs(c.mean() - rho * kb) < 0.1 * rho * kb
    o = ops.block_sparse_attn(q, k, ops.pack_v(v), index, count)
    torch.cuda.synchronize()
    _check_sampled(o, q, k, v, index, count, _sample(T // 128, 4, T), T)
