"""Kernel 1 (pooling, innovation, pooled softmax) vs the oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import pooling as OP
from oracle import selector as OS

pytestmark = pytest.mark.gpu


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _bf16_close(gpu, ref):
    """Pooled means may differ by one bf16 rounding of the fp32 sum."""
    gpu = gpu.float().cpu().numpy()
    tol = np.abs(ref) * 2.0 ** -7 + 1e-30
    bad = np.abs(gpu - ref) > tol
    assert not bad.any(), f"{bad.sum()} pooled values off by more than one bf16 ulp"
    return float((gpu != ref).mean())


@pytest.mark.parametrize("nq,nk,B", [(8288, 8288, 1), (1000, 1041, 1), (128, 64, 1), (77, 130, 1), (500, 640, 2)])
def test_pool_qkv_matches_oracle(nq, nk, B):
    from vasc_amd import ops
    H, D = 3, 64
    q, k, v = _rand((B, H, nq, D), 1), _rand((B, H, nk, D), 2), _rand((B, H, nk, D), 3)
    pq, pk, pv, inn = ops.pool_qkv(q.cuda(), k.cuda(), v.cuda())
    diff_frac = [
        _bf16_close(pq, OP.pool_blocks(q.float().numpy(), 128, round_bf16=True)),
        _bf16_close(pk, OP.pool_blocks(k.float().numpy(), 64, round_bf16=True)),
        _bf16_close(pv, OP.pool_blocks(v.float().numpy(), 64, round_bf16=True)),
    ]
    assert max(diff_frac) < 1e-2
    # innovation is bit-exact given the pooled values the kernel produced
    expect = OS.innovation(pv.float().cpu().numpy())
    assert inn.shape == expect.shape
    assert np.array_equal(inn.cpu().numpy().view(np.uint32), expect.view(np.uint32))


def test_pool_strided_views():
    from vasc_amd import ops
    B, T, H, D = 1, 700, 4, 64
    qkv = _rand((B, T, 3, H, D), 4).cuda()
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    a = ops.pool_qkv(q, k, v)
    b = ops.pool_qkv(q.contiguous(), k.contiguous(), v.contiguous())
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x.view(torch.int32),
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y.view(torch.int32))


@pytest.mark.parametrize("kb", [130, 131, 1, 2, 518])
def test_pair_innovation_bit_exact(kb):
    from vasc_amd import ops
    rng = np.random.default_rng(kb)
    pv = rng.standard_normal((2, 3, kb, 64)).astype(np.float32)
    pv[0, 0, 0, :3] = [np.nan, np.inf, -np.inf]
    if kb >= 2:
        pv[1, 2, 0] = 1e-20  # squares of the differences are float32 denormals
        pv[1, 2, 1] = 3e-20
    out = ops.pair_innovation(torch.from_numpy(pv).cuda()).cpu().numpy()
    expect = OS.innovation(pv)
    assert np.array_equal(out.view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("qb,kb", [(65, 130), (259, 518), (3, 33), (1, 1)])
def test_pooled_softmax(qb, kb):
    from vasc_amd import ops
    B, H = 1, 4
    pq, pk = _rand((B, H, qb, 64), 5) * 4, _rand((B, H, kb, 64), 6) * 4
    pq, pk = pq.to(torch.bfloat16), pk.to(torch.bfloat16)
    # exact fp32 logits path: tight tolerance
    p32 = ops.pooled_softmax(pq.cuda(), pk.cuda(), round_bf16=False).cpu().numpy()
    ref32 = OP.softmax(OP.pooled_logits(pq.float().numpy(), pk.float().numpy(), bf16=False))
    assert np.allclose(p32, ref32, rtol=2e-5, atol=1e-9)
    assert np.allclose(p32.sum(-1), 1.0, atol=1e-5)
    # bf16-rounded logits (the reference's autocast path): a float32 dot
    # product that lands on the other side of a bf16 rounding boundary moves
    # its logit by one bf16 step; every entry must stay inside the bound that
    # this allows (no exceptions)
    p16 = ops.pooled_softmax(pq.cuda(), pk.cuda(), round_bf16=True).cpu().numpy()
    out = OP.prob_outside_bound(p16, pq.float().numpy(), pk.float().numpy(), bf16=True)
    assert not out.any(), f"{out.sum()} of {out.size} outside the one-step logit bound"
    ref16 = OP.softmax(OP.pooled_logits(pq.float().numpy(), pk.float().numpy(), bf16=True))
    assert np.isclose(p16, ref16, rtol=2e-5, atol=1e-9).mean() > 0.99


@pytest.mark.parametrize("qb,kb", [(40, 256), (70, 257), (33, 1280), (33, 1281), (9, 2082)])
def test_pooled_softmax_paths_and_priority(qb, kb):
    """Both launch shapes (one launch up to 1280 key blocks, the two-kernel
    path beyond) stay inside the element-wise bound, and the priority output
    is the cleaned probability, bit for bit."""
    from vasc_amd import ops
    pq, pk = _rand((1, 2, qb, 64), kb) * 3, _rand((1, 2, kb, 64), kb + 1) * 3
    prob, prio = ops.pooled_softmax(pq.cuda(), pk.cuda(), priority=True)
    prob, prio = prob.cpu(), prio.cpu()
    out = OP.prob_outside_bound(prob.numpy(), pq.float().numpy(), pk.float().numpy(), bf16=True)
    assert not out.any(), f"{out.sum()} of {out.size} outside the one-step logit bound"
    assert np.allclose(prob.sum(-1).numpy(), 1.0, atol=1e-5)
    assert torch.equal(prio.view(torch.int32), torch.where(prob > 0, prob, 0.0).view(torch.int32))
    assert torch.equal(ops.pooled_softmax(pq.cuda(), pk.cuda()).cpu().view(torch.int32), prob.view(torch.int32))


def _softmax_ref(pq, pk, scale, rnd):
    dots = np.einsum("...qd,...kd->...qk", pq.float().numpy().astype(np.float64),
                     pk.float().numpy().astype(np.float64)).astype(np.float32)
    if rnd:
        logits = OP.bf16_round((OP.bf16_round(dots) * np.float32(scale)).astype(np.float32))
    else:
        logits = (dots.astype(np.float64) * scale).astype(np.float32)
    return OP.softmax(logits), logits


@pytest.mark.parametrize("case", ["huge", "tiny", "mixed"])
def test_pooled_softmax_extreme_rows(case):
    """Rows whose sum of exp(logit) overflows or underflows the fast pass take
    the online (max, sum) pass; a strip without such rows stays on the fast
    pass in the same launch."""
    from vasc_amd import ops
    qb, kb = 64, 200
    g = torch.Generator().manual_seed(11)
    pk = torch.randn(1, 2, kb, 64, generator=g) * 0.5 + 2.0  # keys share a positive direction
    pq = torch.randn(1, 2, qb, 64, generator=g) * 0.5
    if case == "huge":
        pq += 12.0  # logits ~ +190: exp overflows fp32
    elif case == "tiny":
        pq -= 12.0  # logits ~ -190: exp underflows fp32
    else:
        pq[:, :, :16] += 12.0  # strip 0 partly extreme, strip 1 ordinary
        pq[:, 1, 5] -= 24.0
    pq, pk = pq.to(torch.bfloat16), pk.to(torch.bfloat16)
    for rnd in (False, True):
        got = ops.pooled_softmax(pq.cuda(), pk.cuda(), round_bf16=rnd).cpu().numpy()
        assert np.isfinite(got).all()
        # fp32 logits of magnitude L carry an absolute error of a few ulp(L),
        # which becomes a relative error of the probabilities; bf16 logits may
        # sit one bf16 step away (every entry inside the bound)
        out = OP.prob_outside_bound(got, pq.float().numpy(), pk.float().numpy(), 0.125, bf16=rnd)
        assert not out.any(), f"round={rnd}: {out.sum()} of {out.size} outside the bound"
        assert np.allclose(got.sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("scale", [0.1, 0.125, 1.0])
def test_pooled_softmax_scale(scale):
    """Any scale: a power of two folds into the exp2 argument, others round twice."""
    from vasc_amd import ops
    qb, kb = 70, 96
    pq, pk = _rand((1, 3, qb, 64), 21) * 2, _rand((1, 3, kb, 64), 22) * 2
    for rnd in (False, True):
        got = ops.pooled_softmax(pq.cuda(), pk.cuda(), scale=scale, round_bf16=rnd).cpu().numpy()
        ref, _ = _softmax_ref(pq, pk, scale, rnd)
        if not rnd:
            assert np.isclose(got, ref, rtol=2e-5, atol=1e-9).all()
        out = OP.prob_outside_bound(got, pq.float().numpy(), pk.float().numpy(), scale, bf16=rnd)
        assert not out.any(), f"round={rnd}: {out.sum()} of {out.size} outside the bound"


@pytest.mark.parametrize("nq,nk", [(1000, 1041), (128, 64), (77, 130), (8288, 8328)])
def test_pool_qk_max_bit_exact(nq, nk):
    """Block maxima are exact: bit-identical to the oracle, also for negative
    values and the ragged tail blocks (missing tokens never win)."""
    from vasc_amd import ops
    q, k = (_rand((2, 3, n, 64), s) - 2.0 for n, s in ((nq, 5), (nk, 6)))
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    pq, pk = ops.pool_qk_max(q.cuda(), k.cuda().transpose(1, 2).contiguous().transpose(1, 2))
    assert np.array_equal(pq.float().cpu().numpy(), OP.max_pool_blocks(q.float().numpy(), 128))
    assert np.array_equal(pk.float().cpu().numpy(), OP.max_pool_blocks(k.float().numpy(), 64))
