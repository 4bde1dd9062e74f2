"""The drop-in operator API (vasc_amd.sparse_wrapper / attention) on the GPU.

Covers the reference's own GPU smoke scenario (tests/gpu_smoke.py:14-42:
topk and vasc x 3 layers, [1,2,512,64], s=0.75) and checks every API call
against the oracle on the same inputs: masks and ledger bit-exact, attention
within max-abs 2e-2 / mean-abs 2e-3.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import pooling as OP
from oracle import selector as OS

pytestmark = pytest.mark.gpu


@pytest.fixture
def release_env(request):
    from vasc_amd.launcher import method_environment
    saved = {k: v for k, v in os.environ.items() if k.startswith("SPARSE_VGGT_")}
    for k in saved:
        del os.environ[k]

    def set_mode(model, mode):
        for k in [k for k in os.environ if k.startswith("SPARSE_VGGT_")]:
            del os.environ[k]
        os.environ.update(method_environment(model, mode))

    yield set_mode
    for k in [k for k in os.environ if k.startswith("SPARSE_VGGT_")]:
        del os.environ[k]
    os.environ.update(saved)


def _softmax_rows(rng, shape):
    x = rng.standard_normal(shape)
    return (np.exp(x) / np.exp(x).sum(-1, keepdims=True)).astype(np.float32)


def _bits(t):
    return np.ascontiguousarray(t.detach().float().cpu().numpy()).view(np.uint32)


def test_reference_gpu_smoke_scenario(release_env):
    from vasc_amd.attention import predict_attention
    from vasc_amd.sparse_wrapper import block_sparse_attn_cuda
    torch.manual_seed(0)
    for mode in ("topk", "vasc"):
        release_env("vggt", mode)
        state = {}
        for layer in range(3):
            q, k, v = [torch.randn(1, 2, 512, 64, device="cuda", dtype=torch.float16) for _ in range(3)]
            score = predict_attention(q, k)
            out, sparsity = block_sparse_attn_cuda(q, k, v, score, sparse_ratio=.75, num_patch_tokens=512,
                                                   layer_idx=layer, routing_state=state, return_sparsity=True)
            assert out.shape == q.shape and out.dtype == q.dtype
            assert torch.isfinite(out).all() and out.float().abs().sum() > 0
            assert abs(float(sparsity) - 0.75) < 1e-6  # 2 of 8 blocks, no sink
            # attention equals the oracle on the lists the selector produced
            lists = OS.topk_block_mask(score.cpu().numpy(), 0, sparse_ratio=.75) if mode == "topk" else None
            if lists is not None:
                idx, cnt = OS.index_lists(lists)
                ref = OA.block_sparse_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                                v.float().cpu().numpy(), idx, cnt)
                qb = q.to(torch.bfloat16).float().cpu().numpy()
                ref_bf = OA.block_sparse_attention(qb, k.to(torch.bfloat16).float().cpu().numpy(),
                                                   v.to(torch.bfloat16).float().cpu().numpy(), idx, cnt)
                err = np.abs(out.float().cpu().numpy() - ref_bf)
                assert err.max() <= 2e-2 and err.mean() <= 2e-3
                assert np.abs(ref - ref_bf).max() < 5e-2
        if mode == "vasc":
            assert state["cosa_value_risk_pair_pending_layer"] == 2


def test_predict_attention_matches_oracle():
    from vasc_amd.attention import predict_attention
    g = torch.Generator().manual_seed(1)
    q = (torch.randn(1, 3, 1000, 64, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(1, 3, 1041, 64, generator=g) * 2).to(torch.bfloat16)
    from vasc_amd import ops
    p = predict_attention(q.cuda(), k.cuda()).cpu().numpy()
    ref, rq, rk = OP.pooled_prob(q.float().numpy(), k.float().numpy(), bf16=True)
    assert p.shape == ref.shape
    # the kernel's pooled means are within one bf16 rounding of the oracle's,
    # and its probabilities inside the one-step logit bound around the oracle's
    # softmax of those means, on every entry
    pq, pk, _, _ = ops.pool_qkv(q=q.cuda(), k=k.cuda(), innovation=False)
    pq, pk = pq.float().cpu().numpy(), pk.float().cpu().numpy()
    assert (np.abs(pq - rq) <= np.abs(rq) * 2.0 ** -7).all() and (np.abs(pk - rk) <= np.abs(rk) * 2.0 ** -7).all()
    out = OP.prob_outside_bound(p, pq, pk)
    assert not out.any(), f"{out.sum()} of {out.size} outside the bound"
    assert np.isclose(p, ref, rtol=1e-4, atol=1e-9).mean() > 0.99


def test_predict_attention_max_pooling_matches_oracle():
    from vasc_amd.attention import predict_attention
    g = torch.Generator().manual_seed(2)
    q = (torch.randn(1, 3, 1000, 64, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(1, 3, 1041, 64, generator=g) * 2).to(torch.bfloat16)
    p = predict_attention(q.cuda(), k.cuda(), pool_mode="max").cpu().numpy()
    ref, pq, pk = OP.pooled_prob(q.float().numpy(), k.float().numpy(), bf16=True, pool_mode="max")
    assert p.shape == ref.shape
    # block maxima are exact, so the oracle's pooled inputs are the kernel's
    out = OP.prob_outside_bound(p, pq, pk)
    assert not out.any(), f"{out.sum()} of {out.size} outside the bound"


def test_get_block_mask_bit_exact():
    from vasc_amd.sparse_wrapper import get_block_mask
    rng = np.random.default_rng(2)
    s = rng.integers(0, 5, (1, 4, 65, 130)).astype(np.float32) / 4  # heavy ties
    m = get_block_mask(torch.from_numpy(s).cuda(), 1, sparse_ratio=0.75).cpu().numpy()
    assert np.array_equal(m, OS.topk_block_mask(s, 1, sparse_ratio=0.75))
    m = get_block_mask(torch.from_numpy(s).cuda(), 0, topk=0).cpu().numpy()
    assert np.array_equal(m, OS.topk_block_mask(s, 0, topk=0))


def test_cosa_mask_api_chain_bit_exact(release_env):
    from vasc_amd import sparse_wrapper as SW
    release_env("pi3", "vasc")  # QK-admission service, as the reference's check_selector sets it
    rng = np.random.default_rng(3)
    st_gpu, st_ref = {}, {}
    B, H, Q, K = 1, 2, 9, 31
    for layer in range(6):
        x = rng.standard_normal((B, H, Q, K))
        s = (np.exp(x) / np.exp(x).sum(-1, keepdims=True)).astype(np.float32)
        pv = rng.standard_normal((B, H, K, 64)).astype(np.float32)
        cap = rng.integers(0, K + 1, (B, H, Q))
        base = np.arange(K) < cap[..., None]
        prot = np.zeros_like(base)
        prot[..., -1] = cap > 0
        got = SW.get_cosa_value_risk_pair_debt_mask(
            torch.from_numpy(s).cuda(), torch.from_numpy(pv).cuda(), torch.from_numpy(base).cuda(),
            layer_idx=layer, routing_state=st_gpu, protected_mask=torch.from_numpy(prot).cuda(),
            fp32_projection=True)
        ref, info = OS.cosa_select(s, pv, cap, layer_idx=layer, state=st_ref, protected=prot)
        assert np.array_equal(got.cpu().numpy(), ref)
        assert np.array_equal(_bits(st_gpu[SW.STATE_KEY]), np.asarray(st_ref[OS.STATE_KEY], np.float32).view(np.uint32))
        assert np.array_equal(_bits(st_gpu[SW.PENDING_KEY]), st_ref[OS.PENDING_KEY].view(np.uint32))
        assert np.array_equal(_bits(st_gpu["cosa_value_risk_pair_priority"]), info["priority"].view(np.uint32))
        assert np.array_equal(st_gpu["cosa_value_risk_pair_selected_indices"].cpu().numpy(),
                              st_ref["cosa_value_risk_pair_selected_indices"])
        assert np.array_equal(st_gpu["cosa_value_risk_pair_qk_order_priority"].cpu().numpy(),
                              np.asarray(st_ref["cosa_value_risk_pair_qk_order_priority"], np.float32))
    t_gpu = SW.finalize_cosa_value_risk_pair_debt(st_gpu)
    t_ref = OS.finalize(st_ref)
    assert t_gpu and t_ref and SW.finalize_cosa_value_risk_pair_debt(st_gpu) == {}
    assert np.array_equal(_bits(st_gpu[SW.STATE_KEY]), np.asarray(st_ref[OS.STATE_KEY], np.float32).view(np.uint32))


@pytest.mark.parametrize("model", ["vggt", "pi3"])
def test_block_sparse_attn_c1_end_to_end(release_env, model):
    """Config 1 (8 frames x 1041 tokens, H=16; N(0,1) plus the per-frame
    rank-8 component of scale 0.5) through block_sparse_attn_cuda in vasc
    mode, two chained layers; VGGT uses the official mask (no forced tail),
    Pi3 protects the mixed tail block. The vasc-vs-dense difference of the
    output is reported beside the parity check."""
    import bench
    from vasc_amd import ops
    from vasc_amd.attention import predict_attention
    from vasc_amd.sparse_wrapper import block_sparse_attn_cuda
    release_env(model, "vasc")
    N, P, S, H, D = 8, 1041, 5, 16, 64
    Np, Tk = N * (P - S), N * P
    st_gpu, st_ref = {}, {}
    for layer in range(2):
        q, k, v = bench.synthetic_layer(N, P, S, H, D, seed=4 + layer, device="cpu")
        qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
        score = predict_attention(qc, kc[:, :, :Np])
        out, sparsity = block_sparse_attn_cuda(qc, kc, vc, score, sparse_ratio=0.75, return_sparsity=True,
                                               layer_idx=layer, routing_state=st_gpu, num_patch_tokens=Np)
        from vasc_amd import ops
        _, _, _, iota = ops.pool_qkv(v=vc[:, :, :Np])
        final, _ = OS.layer_selection(score.cpu().numpy(), mode="vasc", sparse_ratio=0.75, patch_tokens=Np,
                                      total_tokens=Tk, official_mask=(model == "vggt"), state=st_ref,
                                      layer_idx=layer, iota=iota.cpu().numpy())
        idx, cnt = OS.index_lists(final)
        assert abs(float(sparsity) - (1 - final.mean())) < 1e-6
        ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
        err = np.abs(out.float().cpu().numpy() - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
        dense = ops.dense_attn(qc, kc, ops.pack_v(vc)).float()
        gap = (out.float() - dense).abs()
        rel = float((out.float() - dense).norm() / dense.norm())
        print(f"C1 {model} layer {layer}: vasc vs dense max-abs {float(gap.max()):.4f}, mean-abs "
              f"{float(gap.mean()):.5f}, relative L2 {rel:.4f}, sparsity {float(sparsity):.4f}")
        assert math.isfinite(rel)
        assert np.array_equal(_bits(st_gpu["cosa_value_risk_pair_debt"]),
                              np.asarray(st_ref[OS.STATE_KEY], np.float32).view(np.uint32))
        kb = -(-Np // 64)
        _check_selected_indices(st_gpu, st_ref, final, kb, int(kb * 0.25) + int(model == "pi3"))


def _check_selected_indices(state, ref_state, final, kb, M):
    """routing_state's execution priority and selected indices: width M (the
    capacity hint, as the reference's ``max_patch_blocks``), the M largest
    priorities of each row in descending order (``priority.topk(M,
    sorted=True)``, int64), bit-exact with the oracle; the first ``count``
    of them are the row's kept patch blocks."""
    assert np.array_equal(_bits(state["cosa_value_risk_pair_priority"]),
                          np.asarray(ref_state["cosa_value_risk_pair_priority"], np.float32).view(np.uint32))
    got = state["cosa_value_risk_pair_selected_indices"].cpu().numpy()
    assert state["cosa_value_risk_pair_max_patch_blocks"] == M and got.shape == final.shape[:-1] + (M,)
    assert got.dtype == np.int64
    assert np.array_equal(got, ref_state["cosa_value_risk_pair_selected_indices"])
    kept = final[..., :kb]
    cnt = kept.sum(-1)
    rows_got, rows_kept = got.reshape(-1, M), kept.reshape(-1, kb)
    for r, c in enumerate(cnt.reshape(-1)):
        assert np.array_equal(np.sort(rows_got[r, :c]), np.flatnonzero(rows_kept[r])), r


@pytest.mark.parametrize("model,mode", [("pi3", "topk"), ("pi3", "vasc"), ("vggt", "vasc")])
def test_block_sparse_attn_c1_cdf_threshold(release_env, model, mode):
    """Config 1 through block_sparse_attn_cuda with a cdf threshold (and a
    ratio lower bound for Pi3 top-k): the sparsity equals the oracle's block
    map, attention is within tolerance on the oracle's lists and the VASC
    ledger matches bit for bit."""
    from vasc_amd import ops
    from vasc_amd.attention import predict_attention
    from vasc_amd.sparse_wrapper import block_sparse_attn_cuda
    release_env(model, mode)
    N, P, S, H, D = 8, 1041, 5, 16, 64
    Np, Tk = N * (P - S), N * P
    ratio = 0.9 if mode == "topk" else None
    g = torch.Generator().manual_seed(6)
    st_gpu, st_ref = {}, {}
    for layer in range(2):
        q = torch.randn(1, H, Np, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
        qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
        score = predict_attention(qc, kc[:, :, :Np])
        out, sparsity = block_sparse_attn_cuda(qc, kc, vc, score, sparse_ratio=ratio, cdf_threshold=0.5,
                                               return_sparsity=True, layer_idx=layer, routing_state=st_gpu,
                                               num_patch_tokens=Np)
        _, _, _, iota = ops.pool_qkv(v=vc[:, :, :Np])
        final, _ = OS.layer_selection(score.cpu().numpy(), mode=mode, sparse_ratio=ratio, cdf_threshold=0.5,
                                      patch_tokens=Np, total_tokens=Tk, official_mask=(model == "vggt"),
                                      state=st_ref, layer_idx=layer, iota=iota.cpu().numpy())
        idx, cnt = OS.index_lists(final)
        assert abs(float(sparsity) - (1 - final.mean())) < 1e-6
        ref = OA.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), idx, cnt)
        err = np.abs(out.float().cpu().numpy() - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
        if mode == "vasc":
            assert np.array_equal(_bits(st_gpu["cosa_value_risk_pair_debt"]),
                                  np.asarray(st_ref[OS.STATE_KEY], np.float32).view(np.uint32))


def test_pv_execution_service_domain_chain(release_env):
    """DEBT_SERVICE_DOMAIN=pv_execution (the reference's default): the
    selector leaves the service to the attention launch, so a second selector
    call without attention in between fails as the reference's does; through
    block_sparse_attn_cuda the observed PV-execution service (every wave
    executes every listed block, threshold inert) drives the same ledger bits
    as the oracle's."""
    from vasc_amd import ops
    from vasc_amd import sparse_wrapper as SW
    from vasc_amd.attention import predict_attention
    release_env("pi3", "vasc")
    os.environ["SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN"] = "pv_execution"
    rng = np.random.default_rng(8)
    s = torch.from_numpy(_softmax_rows(rng, (1, 2, 9, 31))).cuda()
    pv = torch.from_numpy(rng.standard_normal((1, 2, 31, 64)).astype(np.float32)).cuda()
    base = torch.ones(1, 2, 9, 31, dtype=torch.bool, device="cuda")
    st = {}
    SW.get_cosa_value_risk_pair_debt_mask(s, pv, base, layer_idx=0, routing_state=st, fp32_projection=True)
    assert SW.SERVICE_KEY not in st
    with pytest.raises(RuntimeError, match="PV service identity"):
        SW.get_cosa_value_risk_pair_debt_mask(s, pv, base, layer_idx=1, routing_state=st, fp32_projection=True)

    N, P, S, H, D = 4, 1041, 5, 16, 64
    Np, Tk = N * (P - S), N * P
    g = torch.Generator().manual_seed(9)
    st_gpu, st_ref = {}, {}
    for layer in range(3):
        q = torch.randn(1, H, Np, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, H, Tk, D, generator=g).to(torch.bfloat16)
        qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
        score = predict_attention(qc, kc[:, :, :Np])
        SW.block_sparse_attn_cuda(qc, kc, vc, score, sparse_ratio=0.75, layer_idx=layer, routing_state=st_gpu,
                                  num_patch_tokens=Np)
        obs = st_gpu[SW.SERVICE_KEY]
        assert obs["identity_observed"] and obs["layer_idx"] == layer and "service_domain" not in obs
        _, _, _, iota = ops.pool_qkv(v=vc[:, :, :Np])
        final, _ = OS.layer_selection(score.cpu().numpy(), mode="vasc", sparse_ratio=0.75, patch_tokens=Np,
                                      total_tokens=Tk, official_mask=False, state=st_ref, layer_idx=layer,
                                      iota=iota.cpu().numpy())
        Kb = score.shape[-1]
        ex = np.broadcast_to(final[:, :, :, None, :Kb], final.shape[:3] + (4, Kb))
        assert np.array_equal(_bits(obs["pair_service_fraction"][:, :, 0]),
                              OS.pv_execution_service(ex, Kb).view(np.uint32))
        assert np.array_equal(_bits(st_gpu["cosa_value_risk_pair_debt"]),
                              np.asarray(st_ref[OS.STATE_KEY], np.float32).view(np.uint32))
    assert SW.finalize_cosa_value_risk_pair_debt(st_gpu)


def test_pv_post_cut_service_through_block_sparse_attn(release_env, monkeypatch):
    """A finite PV threshold (natural_gap, 6 log2 units) in vasc mode with the
    PV-execution domain, on graded data (every key block's logits sit at a
    multiple of 4 log2 units, so no decision is near the threshold): the
    kernel's execution map equals the oracle's decisions on the lists
    block_sparse_attn_cuda launched, and the observed service is the oracle's
    exact reduction of that map, bit for bit, over two chained layers."""
    from vasc_amd import ops
    from vasc_amd import sparse_wrapper as SW
    from vasc_amd.attention import predict_attention
    release_env("pi3", "vasc")
    os.environ["SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN"] = "pv_execution"
    os.environ["SPARSE_VGGT_QK_PV_THRESHOLD"] = f"natural_gap:{6.0 / math.log2(math.e)!r}"
    captured = {}
    launch = ops.block_sparse_attn_pv

    def spy(q, k, vt, index, count, thr, **kw):
        o, m = launch(q, k, vt, index, count, thr, **kw)
        captured.update(index=index.cpu().numpy(), count=count.cpu().numpy(), thr=thr, map=m.cpu().numpy())
        return o, m

    monkeypatch.setattr(ops, "block_sparse_attn_pv", spy)
    N, P, S, H, D = 4, 1041, 5, 4, 64
    Np, Tk = N * (P - S), N * P
    c = D ** -0.5 * math.log2(math.e)
    rng = np.random.default_rng(12)
    st = {}
    for layer in range(2):
        q = torch.from_numpy(rng.standard_normal((1, H, Np, D)) * 0.01).float()
        q[..., 0] += 1.0
        k = torch.from_numpy(rng.standard_normal((1, H, Tk, D)) * 0.01).float()
        lv = rng.choice([0.0, 4.0, 8.0, 12.0], size=(1, H, math.ceil(Tk / 64)))
        k[..., 0] += torch.from_numpy(np.repeat(lv, 64, axis=-1)[..., :Tk] / c).float()
        v = torch.from_numpy(rng.standard_normal((1, H, Tk, D))).float()
        q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
        qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
        score = predict_attention(qc, kc[:, :, :Np])
        SW.block_sparse_attn_cuda(qc, kc, vc, score, sparse_ratio=0.75, layer_idx=layer, routing_state=st,
                                  num_patch_tokens=Np)
        assert abs(captured["thr"] - 6.0) < 1e-9
        _, _, ref_map = OA.pv_post_cut(q.float().numpy(), k.float().numpy(), captured["index"],
                                       captured["count"], 6.0)
        assert np.array_equal(captured["map"], ref_map), layer
        assert ref_map.sum() < 4 * captured["count"].sum()  # the cut skipped blocks
        Kb = score.shape[-1]
        ref = OS.pv_execution_service(ref_map.reshape(1, H, -1, 4, ref_map.shape[-1]), Kb)
        obs = st[SW.SERVICE_KEY]
        assert np.array_equal(_bits(obs["pair_service_fraction"][:, :, 0]), ref.view(np.uint32)), layer
    assert SW.finalize_cosa_value_risk_pair_debt(st)


def test_global_layer_pv_path_matches_release_path():
    """A finite PV threshold that never cuts (1e9 log2 units) sends the layer
    through the PV post-cut attention instance, the separate special-query
    launch and the restore kernel; the release threshold (1e10, inert) through
    the one token-major launch. Both give the same layer output, bit for bit."""
    from vasc_amd.attention import adaptive_sparse_attention_forward

    class Attn(torch.nn.Module):
        def __init__(self, dim, heads):
            super().__init__()
            self.qkv = torch.nn.Linear(dim, 3 * dim)
            self.proj = torch.nn.Linear(dim, dim)
            self.q_norm = torch.nn.LayerNorm(dim // heads)
            self.k_norm = torch.nn.LayerNorm(dim // heads)
            self.rope = None
            self.heads = heads

    torch.manual_seed(6)
    N, Hp, Wp, S, heads, dim = 3, 10, 13, 5, 4, 256
    P = Hp * Wp + S
    m = Attn(dim, heads).cuda().to(torch.bfloat16)
    x = torch.randn(1, N * P, dim, device="cuda", dtype=torch.bfloat16)
    ys, xs = torch.meshgrid(torch.arange(Hp), torch.arange(Wp), indexing="ij")
    patch_pos = torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1
    pos = torch.cat([torch.zeros(S, 2, dtype=torch.long), patch_pos]).expand(N, P, 2).cuda()
    saved = {k: os.environ.pop(k) for k in list(os.environ) if k.startswith("SPARSE_VGGT_")}
    outs = []
    try:
        for thr in ("1e10", "1e9"):
            os.environ["SPARSE_VGGT_OFFICIAL_MASK"] = "1"
            os.environ["SPARSE_VGGT_QK_PV_THRESHOLD"] = thr
            outs.append(adaptive_sparse_attention_forward(m, x, pos, sparse_ratio=0.5, num_special_tokens=S,
                                                          num_heads=heads, routing_state={}))
    finally:
        for k in ("SPARSE_VGGT_OFFICIAL_MASK", "SPARSE_VGGT_QK_PV_THRESHOLD"):
            os.environ.pop(k, None)
        os.environ.update(saved)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_global_layer_forward_dense_limit():
    """adaptive_sparse_attention_forward at sparsity 0 equals dense attention of
    the same module (all key blocks kept)."""
    from vasc_amd.attention import adaptive_sparse_attention_forward

    class Attn(torch.nn.Module):
        def __init__(self, dim, heads):
            super().__init__()
            self.qkv = torch.nn.Linear(dim, 3 * dim)
            self.proj = torch.nn.Linear(dim, dim)
            self.q_norm = torch.nn.LayerNorm(dim // heads)
            self.k_norm = torch.nn.LayerNorm(dim // heads)
            self.rope = None
            self.heads = heads

    torch.manual_seed(5)
    N, Hp, Wp, S, heads, dim = 3, 10, 12, 5, 4, 256
    P = Hp * Wp + S
    m = Attn(dim, heads).cuda().to(torch.bfloat16)
    x = torch.randn(1, N * P, dim, device="cuda", dtype=torch.bfloat16)
    ys, xs = torch.meshgrid(torch.arange(Hp), torch.arange(Wp), indexing="ij")
    patch_pos = torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1
    pos = torch.cat([torch.zeros(S, 2, dtype=torch.long), patch_pos]).expand(N, P, 2).cuda()
    saved = {k: os.environ.pop(k) for k in list(os.environ) if k.startswith("SPARSE_VGGT_")}
    try:
        os.environ["SPARSE_VGGT_OFFICIAL_MASK"] = "1"
        out = adaptive_sparse_attention_forward(m, x, pos, sparse_ratio=0.0, num_special_tokens=S, num_heads=heads,
                                                routing_state={})
    finally:
        os.environ.pop("SPARSE_VGGT_OFFICIAL_MASK", None)
        os.environ.update(saved)
    with torch.no_grad():
        qkv = m.qkv(x).float().reshape(1, N * P, 3, heads, dim // heads).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        q, k = m.q_norm(q.to(torch.bfloat16)).float(), m.k_norm(k.to(torch.bfloat16)).float()
        ref = torch.nn.functional.scaled_dot_product_attention(q, k, v)
        ref = m.proj(ref.transpose(1, 2).reshape(1, N * P, dim).to(torch.bfloat16))
    err = (out.float() - ref.float()).abs()
    assert err.max() < 6e-2 and err.mean() < 6e-3, (err.max().item(), err.mean().item())


def _check_stats(got, ref, where):
    assert set(got) >= set(ref), (where, sorted(set(ref) - set(got)))
    for key, val in ref.items():
        swap = "overlap" in key or "swap" in key
        np.testing.assert_allclose(float(got[key]), val, rtol=1e-5, atol=1e-3 if swap else 1e-6,
                                   err_msg=f"{where} {key}")


def test_routing_stats_match_oracle(release_env):
    """stats_store of get_cosa_value_risk_pair_debt_mask (the reference's 19
    keys with counterfactual statistics on) and of finalize (6 terminal keys)
    on a 6-layer chain where debt accrues, against the oracle's routing_stats
    (pinned to the reference's own statistics by tests/test_golden.py)."""
    from vasc_amd import sparse_wrapper as SW
    release_env("pi3", "vasc")
    rng = np.random.default_rng(13)
    st_gpu, st_ref = {}, {}
    B, H, Q, K = 1, 2, 65, 130
    gates = []
    for layer in range(6):
        s = _softmax_rows(rng, (B, H, Q, K))
        pv = rng.standard_normal((B, H, K, 64)).astype(np.float32)
        order = np.argsort(-s, axis=-1, kind="stable")
        base = np.zeros((B, H, Q, K), bool)
        np.put_along_axis(base, order[..., :32], True, axis=-1)
        base[..., -1] = True
        prot = np.zeros_like(base)
        prot[..., -1] = True
        cap = base.sum(-1)
        store = {}
        SW.get_cosa_value_risk_pair_debt_mask(
            torch.from_numpy(s).cuda(), torch.from_numpy(pv).cuda(), torch.from_numpy(base).cuda(),
            layer_idx=layer, routing_state=st_gpu, protected_mask=torch.from_numpy(prot).cuda(),
            max_capacity_hint=33, stats_store=store)
        _, info = OS.cosa_select(s, pv, cap, layer_idx=layer, state=st_ref, protected=prot, max_capacity_hint=33)
        gates.append(bool(info["gate"]))
        assert len(store) == 19
        _check_stats(store, OS.routing_stats(info, cap, base, protected=prot), f"layer {layer}")
    assert any(gates) and (np.asarray(st_ref[OS.STATE_KEY]) > 0).any()
    term = {}
    SW.finalize_cosa_value_risk_pair_debt(st_gpu, stats_store=term)
    assert len(term) == 6
    _check_stats(term, OS.finalize(st_ref), "terminal")


def test_layer_routing_stats_store(release_env):
    """block_sparse_attn_cuda with a routing_stats_store in vasc mode (the
    reference passes its base map to the selector and records the resolved
    PV threshold): the selector's statistics equal the oracle's for the same
    layer selection."""
    from vasc_amd.attention import predict_attention
    from vasc_amd.sparse_wrapper import block_sparse_attn_cuda
    release_env("pi3", "vasc")
    torch.manual_seed(4)
    N, P, S = 2, 1041, 5
    n_patch, n_total = N * (P - S), N * P
    state, st_ref = {}, {}
    for layer in range(3):
        q = torch.randn(1, 2, n_patch, 64, device="cuda").to(torch.bfloat16)
        k, v = (torch.randn(1, 2, n_total, 64, device="cuda").to(torch.bfloat16) for _ in range(2))
        score = predict_attention(q, k[:, :, :n_patch])
        store = {}
        block_sparse_attn_cuda(q, k, v, score, sparse_ratio=0.75, num_patch_tokens=n_patch, layer_idx=layer,
                               routing_state=state, routing_stats_store=store)
        from vasc_amd import ops
        iota = ops.pool_qkv(v=v[:, :, :n_patch])[3].cpu().numpy()
        sc = score.cpu().numpy()
        Kb = sc.shape[-1]
        final, info = OS.layer_selection(sc, mode="vasc", sparse_ratio=0.75, patch_tokens=n_patch,
                                         total_tokens=n_total, official_mask=False, state=st_ref, layer_idx=layer,
                                         iota=iota)
        base = OS.topk_block_mask(sc, 0, sparse_ratio=0.75)
        base[..., Kb - 1] = True
        prot = np.zeros_like(base)
        prot[..., Kb - 1] = True
        assert float(store.pop("qk_pv_threshold")) == 1e10
        _check_stats(store, OS.routing_stats(info, base.sum(-1), base, protected=prot), f"layer {layer}")


@pytest.mark.parametrize("pool_mode", ["avg", "max"])
def test_predict_attention_key_block_variance(pool_mode):
    """The variance proxy of predict_attention (ATT:69-89) against the oracle
    (pinned to the reference's own output by tests/test_golden.py)."""
    from vasc_amd.attention import predict_attention
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(1, 3, 1000, 64, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(1, 3, 1041, 64, generator=g) * 2).to(torch.bfloat16)
    prob, var = predict_attention(q.cuda(), k.cuda(), pool_mode=pool_mode, return_key_block_variance=True)
    assert torch.equal(prob, predict_attention(q.cuda(), k.cuda(), pool_mode=pool_mode))
    ref = OP.key_block_variance(k.float().numpy())
    assert var.shape == ref.shape == (1, 3, 17)
    # the pooled bf16 means may differ by one bf16 ulp from a float64-summed mean
    np.testing.assert_allclose(var.cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
