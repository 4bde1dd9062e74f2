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


@pytest.mark.parametrize("nq,nk", [(8288, 8288), (1000, 1041), (128, 64), (77, 130)])
def test_pool_qkv_matches_oracle(nq, nk):
    from vasc_amd import ops
    B, H, D = 1, 3, 64
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
    # bf16-rounded logits (the reference's autocast path): equal except where
    # the fp32 dot product lands on a bf16 rounding boundary
    p16 = ops.pooled_softmax(pq.cuda(), pk.cuda(), round_bf16=True).cpu().numpy()
    ref16 = OP.softmax(OP.pooled_logits(pq.float().numpy(), pk.float().numpy(), bf16=True))
    close = np.isclose(p16, ref16, rtol=2e-5, atol=1e-9)
    assert close.mean() > 0.999, f"{(~close).sum()} of {close.size} differ"
