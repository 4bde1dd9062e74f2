"""Kernel 3 (pack) and kernel 4 (block-sparse / dense attention) vs the oracle.

Tolerance (from the north star): bf16 GPU output vs float64 oracle on the
same bf16 inputs and the same index lists, max-abs <= 2e-2, mean-abs <= 2e-3.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import selector as OS

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _lists(B, H, qb, nkb, seed, density=0.3, allow_empty=False):
    rng = np.random.default_rng(seed)
    counts = rng.binomial(nkb, density, size=(B, H, qb)).clip(0 if allow_empty else 1, nkb)
    idx = np.full((B, H, qb, nkb), -1, np.int32)
    for b in range(B):
        for h in range(H):
            for i in range(qb):
                sel = np.sort(rng.choice(nkb, size=counts[b, h, i], replace=False))
                idx[b, h, i, : sel.size] = sel
    return idx, counts.astype(np.int32)


def _check(out, ref):
    err = np.abs(out.float().cpu().numpy().astype(np.float64) - ref)
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert err.max() <= MAX_ABS, f"max-abs {err.max():.3e}"
    assert err.mean() <= MEAN_ABS, f"mean-abs {err.mean():.3e}"
    return err.max(), err.mean()


def test_pack_v_layout_bit_exact():
    from vasc_amd import ops
    B, H, T, D = 1, 3, 200, 64
    v = _rand((B, H, T, D), 1)
    vt = ops.pack_v(v.cuda()).cpu()
    nkb = math.ceil(T / 64)
    vp = torch.zeros(B, H, nkb * 64, D, dtype=torch.bfloat16)
    vp[:, :, :T] = v
    pos = torch.arange(64)
    s, hh, e = pos // 16, (pos % 16) // 8, pos % 8
    key = 16 * s + 8 * (e // 4) + 4 * hh + (e % 4)
    expect = vp.view(B, H, nkb, 64, D)[:, :, :, key, :].transpose(-1, -2)
    assert torch.equal(vt.view(torch.int16), expect.contiguous().view(torch.int16))


@pytest.mark.parametrize("nq,nk,seed,B", [(128, 64, 0, 1), (300, 200, 1, 1), (1000, 1041, 2, 1), (77, 130, 3, 1),
                                         (300, 330, 4, 2)])
def test_block_sparse_matches_oracle(nq, nk, seed, B):
    from vasc_amd import ops
    H, D = 2, 64
    q, k, v = _rand((B, H, nq, D), seed), _rand((B, H, nk, D), seed + 100), _rand((B, H, nk, D), seed + 200)
    qb, nkb = math.ceil(nq / 128), math.ceil(nk / 64)
    idx, cnt = _lists(B, H, qb, nkb, seed)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    out = ops.block_sparse_attn(qc, kc, ops.pack_v(vc), torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda())
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
    _check(out, ref)


def test_dense_matches_oracle_and_full_lists():
    from vasc_amd import ops
    B, H, nq, nk, D = 1, 2, 520, 777, 64
    q, k, v = _rand((B, H, nq, D), 5), _rand((B, H, nk, D), 6), _rand((B, H, nk, D), 7)
    qc, kc, vt = q.cuda(), k.cuda(), ops.pack_v(v.cuda())
    dense = ops.dense_attn(qc, kc, vt)
    idx, cnt = OA.dense_lists(B, H, nq, nk)
    sparse = ops.block_sparse_attn(qc, kc, vt, torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda())
    assert torch.equal(dense.view(torch.int16), sparse.view(torch.int16))
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
    _check(dense, ref)
    sdpa = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double())
    assert np.abs(sdpa.numpy() - ref).max() < 1e-9


def test_delta_lut_equals_index_lists():
    from vasc_amd import ops
    from oracle import lut as OL
    B, H, nq, nk = 1, 2, 400, 650
    q, k, v = _rand((B, H, nq, 64), 8), _rand((B, H, nk, 64), 9), _rand((B, H, nk, 64), 10)
    qb, nkb = math.ceil(nq / 128), math.ceil(nk / 64)
    idx, cnt = _lists(B, H, qb, nkb, 11)
    mask = np.zeros((B, H, qb, nkb), bool)
    for b in range(B):
        for h in range(H):
            for i in range(qb):
                mask[b, h, i, idx[b, h, i, : cnt[b, h, i]]] = True
    lut, vcnt = OL.encode(mask)
    assert (vcnt == cnt).all()
    qc, kc, vt = q.cuda(), k.cuda(), ops.pack_v(v.cuda())
    a = ops.block_sparse_attn(qc, kc, vt, torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda())
    b = ops.block_sparse_attn(qc, kc, vt, torch.from_numpy(lut).cuda(), torch.from_numpy(vcnt).cuda(), delta=True)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_empty_rows_and_out_of_range_blocks():
    from vasc_amd import ops
    B, H, nq, nk = 1, 1, 256, 256
    q, k, v = _rand((B, H, nq, 64), 12), _rand((B, H, nk, 64), 13), _rand((B, H, nk, 64), 14)
    idx = np.array([[[[1, 3, -1, 99], [0, 0, 0, 0]]]], np.int32)  # row 0: blocks 1,3 + two invalid
    cnt = np.array([[[4, 0]]], np.int32)
    qc, kc, vt = q.cuda(), k.cuda(), ops.pack_v(v.cuda())
    out = ops.block_sparse_attn(qc, kc, vt, torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()).float().cpu()
    assert torch.count_nonzero(out[0, 0, 128:]) == 0
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                    np.array([[[[1, 3], [0, 0]]]], np.int32), np.array([[[2, 0]]], np.int32))
    err = np.abs(out.numpy() - ref)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


def test_strided_inputs_match_contiguous():
    from vasc_amd import ops
    B, H, T, D = 1, 4, 333, 64
    qkv = _rand((B, T, 3, H, D), 15).cuda()
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))  # [B,H,T,D] strided views
    vt = ops.pack_v(v)
    a = ops.dense_attn(q, k, vt)
    b = ops.dense_attn(q.contiguous(), k.contiguous(), ops.pack_v(v.contiguous()))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_c1_layer_topk_lists():
    """Config 1 shape (8 frames x 1041 tokens, H=16) with Top-K lists + sink."""
    from vasc_amd import ops
    N, P, S, H, D = 8, 1041, 5, 16, 64
    Np, Tk = N * (P - S), N * P
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, H, Np, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
    qb, kb = math.ceil(Np / 128), math.ceil(Np / 64)
    score = np.random.default_rng(0).random((1, H, qb, kb)).astype(np.float32)
    final = OS.topk_block_mask(score, math.ceil(Tk / 64) - kb, sparse_ratio=0.75)
    idx, cnt = OS.index_lists(final)
    out = ops.block_sparse_attn(q.cuda(), k.cuda(), ops.pack_v(v.cuda()), torch.from_numpy(idx).cuda(),
                                torch.from_numpy(cnt).cuda())
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
    _check(out, ref)


@pytest.mark.parametrize("case", ["high", "low", "mixed"])
def test_extreme_logits_take_the_exact_path(case):
    """Logits far outside the fast path's range: above 64 in log2 units (the
    block sum overflows 2^64) or all below -126 (every probability would
    underflow). The kernel must move its exponent offset and still match the
    float64 softmax."""
    from vasc_amd import ops
    B, H, nq, nk, D = 1, 2, 256, 640, 64
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, H, nq, D, generator=g)
    k = torch.randn(B, H, nk, D, generator=g)
    v = torch.randn(B, H, nk, D, generator=g)
    u = torch.randn(D, generator=g)
    u = u / u.norm() * 8.0
    if case == "high":
        # logit std ~ 0.18 * 4 * 4 * 8 = 23: row maxima 50..105
        q, k = q * 4.0, k * 4.0
    else:
        # every key ~ -4u: rows ~ +4u sit near -185 (all below -126), rows
        # ~ -4u near +185; "mixed" interleaves those with ordinary rows
        k = -4.0 * u + 0.5 * torch.randn(B, H, nk, D, generator=g)
        low = 4.0 * u + 0.5 * torch.randn(B, H, nq, D, generator=g)
        if case == "low":
            q = low
        else:
            high = -4.0 * u + 0.5 * torch.randn(B, H, nq, D, generator=g)
            r = torch.arange(nq) % 3
            q = torch.where((r == 0).view(1, 1, nq, 1), low, torch.where((r == 1).view(1, 1, nq, 1), high, q))
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    qb, nkb = math.ceil(nq / 128), math.ceil(nk / 64)
    idx, cnt = _lists(B, H, qb, nkb, 22, density=0.6)
    out = ops.block_sparse_attn(q.cuda(), k.cuda(), ops.pack_v(v.cuda()), torch.from_numpy(idx).cuda(),
                                torch.from_numpy(cnt).cuda())
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
    _check(out, ref)
    dense = ops.dense_attn(q.cuda(), k.cuda(), ops.pack_v(v.cuda()))
    dl = OA.dense_lists(B, H, nq, nk)
    _check(dense, OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), *dl))


# ---------------------------------------------------------------- PV post-cut
def _graded_blocks(nq, nk, levels, seed):
    """Query rows a*e0 (+ small noise) and key block j = levels[j] / c * e0
    (+ small noise): block j's logits sit at levels[j] in log2 units, so the
    post-cut decisions have margins of whole log2 units."""
    D = 64
    c = D ** -0.5 * math.log2(math.e)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 2, nq, D, generator=g) * 0.01
    q[..., 0] += 1.0
    k = torch.randn(1, 2, nk, D, generator=g) * 0.01
    for j in range(math.ceil(nk / 64)):
        k[:, :, 64 * j:64 * (j + 1), 0] += float(levels[j % len(levels)]) / c
    v = torch.randn(1, 2, nk, D, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("nq,nk,thr", [(512, 1000, 6.0), (300, 1041, 6.0), (256, 640, [6.0, 1e10])])
def test_pv_post_cut_matches_oracle(nq, nk, thr):
    """Execution map bit-exact with the oracle's decisions; output within
    tolerance of float64 attention over the executed blocks."""
    from vasc_amd import ops
    levels = [0, 8, 4, 12, 0, 4, 8, 0]  # log2 units; with threshold 6 every gap + 6 is >= 2 away from 0
    q, k, v = _graded_blocks(nq, nk, levels, seed=nq)
    qb, nkb = math.ceil(nq / 128), math.ceil(nk / 64)
    idx, cnt = _lists(1, 2, qb, nkb, seed=nk, density=0.6)
    o, pv_map = ops.block_sparse_attn_pv(q.cuda(), k.cuda(), ops.pack_v(v.cuda()), torch.from_numpy(idx).cuda(),
                                         torch.from_numpy(cnt).cuda(), thr)
    ex_idx, ex_cnt, ref_map = OA.pv_post_cut(q.float().numpy(), k.float().numpy(), idx, cnt, thr)
    assert ref_map.sum() < 4 * cnt.sum()  # the cut removed blocks
    assert np.array_equal(pv_map.cpu().numpy(), ref_map)
    ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), ex_idx, ex_cnt)
    _check(o, ref)
