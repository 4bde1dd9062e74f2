"""Pins of the oracle's pooling, LUT, attention, profile and CPU baseline."""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import cpu_baseline as CB
from oracle import lut as OL
from oracle import pooling as OP
from oracle import profile as PR
from oracle import selector as OS


# ------------------------------------------------------------------ pooling
def test_pool_blocks_exact_means_and_tail():
    rng = np.random.default_rng(0)
    x = rng.integers(-50, 50, (1, 1, 150, 3)).astype(np.float32) / 8
    out = OP.pool_blocks(x, 64)
    assert out.shape == (1, 1, 3, 3)
    for b, (lo, hi) in enumerate(((0, 64), (64, 128), (128, 150))):
        for d in range(3):
            exact = sum(Fraction(float(v)) for v in x[0, 0, lo:hi, d]) / (hi - lo)
            assert out[0, 0, b, d] == np.float32(float(exact))


def test_pool_blocks_matches_torch_avg_pool_ceil_mode():
    x = torch.randn(2, 3, 777, 64)
    ours = OP.pool_blocks(x.numpy(), 128)
    ref = torch.nn.functional.avg_pool1d(x.reshape(6, 777, 64).transpose(1, 2), 128, ceil_mode=True)
    np.testing.assert_allclose(ours, ref.transpose(1, 2).reshape(2, 3, -1, 64).numpy(), rtol=1e-5, atol=1e-6)


def test_bf16_round_matches_torch():
    x = torch.randn(10000) * 10 ** torch.randint(-20, 20, (10000,)).float()
    np.testing.assert_array_equal(OP.bf16_round(x.numpy()), x.to(torch.bfloat16).float().numpy())


def test_softmax_rows_sum_to_one():
    p = OP.softmax(np.random.default_rng(1).standard_normal((4, 9)) * 30)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)


# ------------------------------------------------------------------ LUT
def test_lut_encode_matches_reference_restatement_and_round_trips():
    rng = np.random.default_rng(2)
    m = rng.random((2, 3, 7, 40)) < 0.3
    m[0, 0, 0] = False
    m[0, 0, 1] = True
    lut, cnt = OL.encode(m)
    ref_lut, ref_cnt = OL.reference_block_map_lut(m)
    assert np.array_equal(cnt, ref_cnt)
    for idx in np.ndindex(m.shape[:-1]):
        c = cnt[idx]
        assert np.array_equal(lut[idx][:c], ref_lut[idx][:c])
        assert not lut[idx][c:].any()
    assert np.array_equal(OL.decode(lut, cnt), m)


# ------------------------------------------------------------------ attention
def test_block_sparse_attention_matches_masked_sdpa():
    rng = np.random.default_rng(3)
    B, H, Nq, Tk, D = 1, 2, 300, 230, 16
    q, k, v = (rng.standard_normal((B, H, n, D)) for n in (Nq, Tk, Tk))
    qb, kb = 3, 4
    mask_blocks = rng.random((B, H, qb, kb)) < 0.5
    mask_blocks[..., 0] = True
    idx, cnt = OS.index_lists(mask_blocks)
    out = OA.block_sparse_attention(q, k, v, idx, cnt)
    full = np.repeat(np.repeat(mask_blocks, 128, axis=2), 64, axis=3)[:, :, :Nq, :Tk]
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(t) for t in (q, k, v)), attn_mask=torch.from_numpy(full))
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-10)
    # sampled query blocks: those rows equal the full result, every other row is zero
    part = OA.block_sparse_attention(q, k, v, idx, cnt, q_blocks=[2, 0, 2])
    rows = np.r_[0:128, 256:300]
    np.testing.assert_array_equal(part[:, :, rows], out[:, :, rows])
    assert not part[:, :, 128:256].any()


def test_dense_lists_equal_unmasked_attention():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((1, 1, n, 8)) for n in (200, 150, 150))
    idx, cnt = OA.dense_lists(1, 1, 200, 150)
    out = OA.block_sparse_attention(q, k, v, idx, cnt)
    ref = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(t) for t in (q, k, v)))
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-10)


# ------------------------------------------------------------------ profile
def test_structural_profile_matches_release_assertions():
    """The reference's tests/test_release.py:43-51, 109-121."""
    for model, count, low in (("vggt", 24, 11), ("pi3", 18, 12)):
        for s in (.75, .85):
            vals = PR.layer_sparsity(model, s)
            assert len(vals) == count
            assert abs(sum(vals) / count - s) < 1e-9
            assert abs(vals[low] - (s - .05)) < 1e-9
        assert PR.layer_sparsity(model, .65) is None
        assert PR.layer_sparsity(model, .70) is None
        assert PR.layer_sparsity(model, .7001) is not None
        assert PR.layer_sparsity(model, .85, "uniform") is None
        with pytest.raises(ValueError):
            PR.layer_sparsity(model, .99)


def test_budget_table_of_the_configs():
    c2 = PR.layer_sparsity("vggt", .75)
    assert {PR.budget(518, s) for s in c2} == {155, 120}
    c3 = PR.layer_sparsity("vggt", .875)
    assert {PR.budget(2072, s) for s in c3} == {362, 224}
    c4 = PR.layer_sparsity("pi3", .75)
    assert {PR.budget(1036, s) for s in c4} == {310, 233}
    assert PR.budget(130, .75) == 32 and PR.budget(518, .75) == 129


# ------------------------------------------------------------------ CPU baseline
def test_cpu_baseline_matches_float64_oracle():
    g = torch.Generator().manual_seed(5)
    Np, Tk, H, D = 500, 520, 2, 64
    q = torch.randn(1, H, Np, D, generator=g)
    k = torch.randn(1, H, Tk, D, generator=g)
    v = torch.randn(1, H, Tk, D, generator=g)
    out = CB.topk_layer(q, k, v, 0.75)
    prob = CB.pooled_prob(q, k[..., :Np, :])
    sink = -(-Tk // 64) - prob.shape[-1]
    final = OS.topk_block_mask(prob.numpy(), sink, sparse_ratio=0.75)
    idx, cnt = OS.index_lists(final)
    ref = OA.block_sparse_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), idx, cnt)
    np.testing.assert_allclose(out.numpy(), ref, atol=2e-5)


def test_cpu_dense_baseline_matches_float64_oracle():
    g = torch.Generator().manual_seed(6)
    Np, Tk, H, D = 300, 333, 2, 64
    q = torch.randn(1, H, Np, D, generator=g)
    k = torch.randn(1, H, Tk, D, generator=g)
    v = torch.randn(1, H, Tk, D, generator=g)
    out = CB.dense_layer(q, k, v, rows=128)  # several row chunks, a partial last one
    idx, cnt = OA.dense_lists(1, H, Np, Tk)
    ref = OA.block_sparse_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), idx, cnt)
    np.testing.assert_allclose(out.numpy(), ref, atol=2e-5)


# ---------------------------------------------------------------- PV post-cut
def _rank_one(levels, Nq=128, block_k=64, a=1.0):
    """q rows = a * e0, key block j = levels[j] * e0: every logit of block j
    is a * levels[j], so block j's row max is a * levels[j] * D^-0.5 * log2 e."""
    D = 64
    q = np.zeros((1, 1, Nq, D))
    q[..., 0] = a
    k = np.zeros((1, 1, len(levels) * block_k, D))
    for j, lv in enumerate(levels):
        k[0, 0, j * block_k:(j + 1) * block_k, 0] = lv
    return q, k


def _unit():
    return 64 ** -0.5 * np.log2(np.e)  # log2 units per unit logit


def test_pv_post_cut_hand_sequences():
    u = _unit()
    # logits 10, 0, 5 (in units of 1/u) with threshold 6: the first block always runs,
    # 0 is 10 below the running max (skip), 5 is 5 below (runs: -5 + 6 > 0)
    q, k = _rank_one([10 / u, 0.0, 5 / u])
    idx = np.array([[[[0, 1, 2]]]], np.int32)
    lists, cnt, m = OA.pv_post_cut(q, k, idx, np.array([[[3]]]), 6.0)
    assert cnt[0, 0, 0] == 2 and list(lists[0, 0, 0, :2]) == [0, 2]
    assert m[0, 0, :4, 0].all() and not m[0, 0, :, 1].any() and m[0, 0, :4, 2].all()
    # increasing maxima always run; a later low block is judged against the raised max
    q, k = _rank_one([0.0, 10 / u, 3 / u])
    lists, cnt, _ = OA.pv_post_cut(q, k, idx, np.array([[[3]]]), 6.0)
    assert list(lists[0, 0, 0, : cnt[0, 0, 0]]) == [0, 1]
    # list order, not block order: listed as 1, 0, 2 the highest block comes first and
    # both others fall more than 6 below it
    lists, cnt, _ = OA.pv_post_cut(q, k, np.array([[[[1, 0, 2]]]], np.int32), np.array([[[3]]]), 6.0)
    assert list(lists[0, 0, 0, : cnt[0, 0, 0]]) == [1]


def test_pv_post_cut_boundary_inert_and_padded_rows():
    u = _unit()
    q, k = _rank_one([8 / u, 2 / u])
    idx, c1 = np.array([[[[0, 1]]]], np.int32), np.array([[[2]]])
    assert OA.pv_post_cut(q, k, idx, c1, 6.0)[1][0, 0, 0] == 1           # gap -6 + 6 = 0: skipped
    assert OA.pv_post_cut(q, k, idx, c1, 6.0 + 1e-9)[1][0, 0, 0] == 2    # just above: runs
    lists, cnt, m = OA.pv_post_cut(q, k, idx, c1, 1e10)
    assert cnt[0, 0, 0] == 2 and m.sum() == 8
    # query rows past Nq count with zero logits: with all real logits negative,
    # the zero rows set the block maxima
    q, k = _rank_one([-50 / u, -60 / u], Nq=100, a=1.0)
    assert OA.pv_post_cut(q, k, idx, c1, 1.0)[1][0, 0, 0] == 2           # padded rows: 0 and 0, gap 0
    q, k = _rank_one([-50 / u, -60 / u], Nq=128, a=1.0)
    assert OA.pv_post_cut(q, k, idx, c1, 1.0)[1][0, 0, 0] == 1           # no padding: gap -10


def test_max_pool_blocks_matches_torch():
    """``max_pool_blocks`` is F.max_pool1d(kernel, ceil_mode=True) on bf16 data,
    including ragged tails and all-negative blocks."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(3)
    for T, blk in ((1000, 128), (1041, 64), (64, 64), (7, 64)):
        x = (torch.randn(2, 3, T, 64, generator=g) - 3.0).to(torch.bfloat16).float()
        ref = F.max_pool1d(x.reshape(6, T, 64).transpose(1, 2), blk, ceil_mode=True).transpose(1, 2)
        got = OP.max_pool_blocks(x.numpy(), blk)
        assert np.array_equal(got, ref.reshape(2, 3, -1, 64).numpy())


def test_prob_bound_admits_rounding_flips_and_rejects_larger_errors():
    """The pooled-probability tolerance: moving any logit by one bf16 step
    (what a float32 dot product landing on the other side of a rounding
    boundary does) stays inside the bound; a torch float32 matmul with its
    own bf16 roundings stays inside; four steps on one logit, or a softmax
    of a transposed key set, does not."""
    rng = np.random.default_rng(5)
    pq = OP.bf16_round((rng.standard_normal((1, 2, 20, 64)) * 4).astype(np.float32))
    pk = OP.bf16_round((rng.standard_normal((1, 2, 40, 64)) * 4).astype(np.float32))
    logits = OP.pooled_logits(pq, pk)
    ref = OP.softmax(logits)
    assert not OP.prob_outside_bound(ref, pq, pk).any()
    # one bf16 step on the true value's side (below a power of two the gap is half the one above)
    step = OP.bf16_spacing(np.abs(logits) * (1 - 2.0 ** -10)).astype(np.float32)
    flip = np.where(rng.random(logits.shape) < 0.5, -1, 1).astype(np.float32)
    assert not OP.prob_outside_bound(OP.softmax(logits + flip * step), pq, pk).any()
    # the same predictor computed by torch in float32 with the autocast roundings
    dots = torch.from_numpy(pq) @ torch.from_numpy(pk).transpose(-1, -2)
    tl = dots.to(torch.bfloat16).float().mul(0.125).to(torch.bfloat16).float().softmax(-1).numpy()
    assert not OP.prob_outside_bound(tl, pq, pk).any()
    # a planted error of four steps on each row's largest logit is caught on every row
    j = logits.argmax(-1)
    bad = logits.copy()
    np.put_along_axis(bad, j[..., None], np.take_along_axis(logits + 4 * step, j[..., None], -1), -1)
    out = OP.prob_outside_bound(OP.softmax(bad), pq, pk)
    assert out.any(-1).all()
    # so is a predictor that pairs the queries with the wrong keys
    assert OP.prob_outside_bound(OP.softmax(OP.pooled_logits(pq, pk[:, ::-1])), pq, pk).any()


def test_bf16_spacing_is_the_gap_between_neighbours():
    x = torch.tensor([1.0, 1.5, 2.0, 3.0, 0.01, 100.0, -7.0], dtype=torch.bfloat16)
    nxt = torch.nextafter(x.abs(), torch.tensor(float("inf"), dtype=torch.bfloat16))
    assert np.array_equal(OP.bf16_spacing(x.float().numpy()), (nxt.float() - x.abs().float()).numpy())
