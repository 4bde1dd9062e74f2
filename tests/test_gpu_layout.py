"""Kernel 5 (token layout) and the whole-layer attention launch vs the oracle.

Layout without norm/rotation moves bf16 values and is bit-exact. With the
per-head LayerNorm and the 2D rotary embedding the kernel computes in
float32 and rounds once to bf16: within one bf16 rounding of the float64
oracle plus the float32 error (|err| <= 2^-8 |ref| + 1e-5).
Attention tolerances as elsewhere: max-abs 2e-2, mean-abs 2e-3 vs float64.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import layout as OL

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _to_np(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("N,P,S,H", [(3, 1041, 5, 2), (2, 37, 0, 3), (4, 6, 6, 1), (1, 131, 4, 16)])
def test_pack_layout_bit_exact(N, P, S, H):
    from vasc_amd import ops
    D = 64
    qkv = _bf16((1, N * P, 3 * H * D), N * 100 + P)
    x = qkv.cuda().view(1, N * P, 3, H, D)
    qp, qs, k, v = ops.pack_qkv(x[:, :, 0], x[:, :, 1], x[:, :, 2], N, P, S)
    rp, rs, rk, rv = OL.pack_layer(qkv.float().numpy(), N, P, S, H)
    assert np.array_equal(_to_np(qp), rp)
    assert np.array_equal(_to_np(k), rk) and np.array_equal(_to_np(v), rv)
    if S:
        assert np.array_equal(_to_np(qs), rs)
    else:
        assert qs is None


def test_pack_from_head_major_views():
    """q/k/v given as [B,H,T,D] tensors (transposed views) instead of one qkv buffer."""
    from vasc_amd import ops
    N, P, S, H, D = 2, 300, 5, 4, 64
    q, k, v = (_bf16((2, H, N * P, D), s) for s in (1, 2, 3))
    qp, qs, ko, vo = ops.pack_qkv(*(t.cuda().transpose(1, 2) for t in (q, k, v)), N, P, S)
    assert np.array_equal(_to_np(qp), OL.get_patch_tokens(q.float().numpy(), N, P, S))
    assert np.array_equal(_to_np(qs), OL.get_special_tokens(q.float().numpy(), N, P, S))
    assert np.array_equal(_to_np(ko), OL.reorder_to_patch_then_special(k.float().numpy(), N, P, S))
    assert np.array_equal(_to_np(vo), OL.reorder_to_patch_then_special(v.float().numpy(), N, P, S))


@pytest.mark.parametrize("which", ["both", "q_only", "k_only"])
def test_pack_norm_and_rotary(which):
    """Per-head LayerNorm of q and/or k, then the 2D rotary embedding, against
    the oracle (the LayerNorm weights are staged per workgroup, so the
    one-sided cases check that the other tensor's rows stay untouched)."""
    from vasc_amd import ops
    from vasc_amd.aggregator import RotaryPositionEmbedding2D
    N, Hp, Wp, S, H, D = 3, 9, 13, 5, 2, 64
    P = Hp * Wp + S
    qkv = _bf16((1, N * P, 3 * H * D), 7, 2.0)
    g = torch.Generator().manual_seed(8)
    qw, qb, kw = (torch.randn(D, generator=g) for _ in range(3))
    ys, xs = torch.meshgrid(torch.arange(Hp), torch.arange(Wp), indexing="ij")
    frame_pos = torch.cat([torch.zeros(S, 2, dtype=torch.long), torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1])
    pos = frame_pos.repeat(N, 1)  # [T, 2]
    cos, sin = RotaryPositionEmbedding2D().tables(D, "cuda")
    x = qkv.cuda().view(1, N * P, 3, H, D)
    use_q, use_k = which in ("both", "q_only"), which in ("both", "k_only")
    qp, qs, k, v = ops.pack_qkv(x[:, :, 0], x[:, :, 1], x[:, :, 2], N, P, S,
                                q_norm=(qw.cuda(), qb.cuda(), 1e-6) if use_q else None,
                                k_norm=(kw.cuda(), None, 1e-5) if use_k else None, pos=pos.cuda(),
                                rope_tables=(cos, sin))
    rp, rs, rk, rv = OL.pack_layer(qkv.float().numpy(), N, P, S, H,
                                   q_norm=(qw.numpy(), qb.numpy(), 1e-6) if use_q else None,
                                   k_norm=(kw.numpy(), None, 1e-5) if use_k else None, pos=pos.numpy(),
                                   tables=(cos.cpu().numpy(), sin.cpu().numpy()))
    for got, ref in ((qp, rp), (qs, rs), (k, rk)):
        err = np.abs(_to_np(got) - ref)
        assert (err <= np.abs(ref) * 2.0 ** -8 + 1e-5).all(), err.max()
    assert np.array_equal(_to_np(v), rv)


@pytest.mark.parametrize("N,P,S,H", [(1, 1041, 0, 16), (3, 70, 5, 3)])
def test_pack_without_v_and_strided_v_tiles(N, P, S, H):
    """pack_qkv with v=None writes the same q and k as the full pack (the row
    space then spans q and k only), and V tiles packed straight from the
    projection's strided rows equal those packed from the packed v (frame
    layers: S = 0, the order unchanged)."""
    from vasc_amd import ops
    D = 64
    qkv = _bf16((2, N * P, 3 * H * D), N * 7 + P).cuda().view(2, N * P, 3, H, D)
    w = torch.randn(D, generator=torch.Generator().manual_seed(3)).cuda()
    full = ops.pack_qkv(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S, q_norm=(w, None, 1e-6))
    part = ops.pack_qkv(qkv[:, :, 0], qkv[:, :, 1], None, N, P, S, q_norm=(w, None, 1e-6))
    assert part[3] is None
    for a, b in zip(full[:3], part[:3]):
        assert (a is None) == (b is None)
        if a is not None:
            assert np.array_equal(_bits(a), _bits(b))
    if S == 0:
        vt_strided = ops.pack_v(qkv[:, :, 2].transpose(1, 2))
        assert np.array_equal(_bits(vt_strided), _bits(ops.pack_v(full[3])))


def _one_bf16_rounding(got, ref):
    """Pooled means within one bf16 rounding of the float64 mean (the
    kernel's float32 sums may round the other way)."""
    got = got.float().cpu().numpy().astype(np.float64)
    bad = np.abs(got - ref) > np.abs(ref) * 2.0 ** -7 + 1e-30
    assert not bad.any(), f"{bad.sum()} pooled values off by more than one bf16 rounding"


@pytest.mark.parametrize("N,P,S,H,B,transform", [
    (3, 1041, 5, 2, 1, True),    # C1-like frames, norm + rotary, ragged tails
    (2, 37, 0, 3, 2, False),     # no special tokens, two batch entries
    (1, 131, 4, 16, 1, True),    # 16 heads, one query block, odd key-block count
    (4, 6, 5, 1, 1, False),      # one patch token per frame
    (2, 69, 5, 2, 1, True),      # patch tokens exactly one query block, special tail block
    (2, 70, 5, 2, 2, False),     # 130 patch tokens: odd key blocks, 2-token tail
    (1, 8192 + 5, 5, 1, 1, True),  # 8192 patch tokens: no tail
])
def test_pack_global_matches_separate_passes(N, P, S, H, B, transform):
    """The fused layout + pooling + V tiles against the separate passes it
    replaces: q_patch, q_special and k bit-identical to pack_qkv, the V tiles
    bit-identical to pack_v of pack_qkv's v, the pooled means within one bf16
    rounding of the float64 block means of the packed patch tokens (the
    oracle's pool_blocks), the innovation bit-exact given the pooled values."""
    from oracle import selector as OS
    from oracle import pooling as OP
    from vasc_amd import ops
    from vasc_amd.aggregator import RotaryPositionEmbedding2D
    D, T = 64, N * P
    qkv = _bf16((B, T, 3 * H * D), N * 31 + P, 2.0).cuda().view(B, T, 3, H, D)
    kw = {}
    if transform:
        g = torch.Generator().manual_seed(P)
        qw, qb, kwt = (torch.randn(D, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
        pos = torch.randint(0, 40, (B, T, 2), generator=g).cuda()
        kw = dict(q_norm=(qw, qb, 1e-6), k_norm=(kwt, None, 1e-5), pos=pos,
                  rope_tables=RotaryPositionEmbedding2D().tables(D, "cuda"))
    sep = ops.pack_qkv(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S, **kw)
    qp, qs, k, vt, pq, pk, inn, pv = ops.pack_global(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S,
                                                     pooled_v=True, **kw)
    assert np.array_equal(_bits(qp), _bits(sep[0]))
    assert (qs is None) == (sep[1] is None)
    if qs is not None:
        assert np.array_equal(_bits(qs), _bits(sep[1]))
    assert np.array_equal(_bits(k), _bits(sep[2]))
    assert np.array_equal(_bits(vt), _bits(ops.pack_v(sep[3])))
    n_patch = N * (P - S)
    _one_bf16_rounding(pq, OP.pool_blocks(_to_np(sep[0]), 128))
    _one_bf16_rounding(pk, OP.pool_blocks(_to_np(sep[2])[:, :, :n_patch], 64))
    _one_bf16_rounding(pv, OP.pool_blocks(_to_np(sep[3])[:, :, :n_patch], 64))
    expect = OS.innovation(pv.float().cpu().numpy())
    assert inn.shape == expect.shape
    assert np.array_equal(inn.cpu().numpy().view(np.uint32), expect.view(np.uint32))
    # without the optional outputs the required ones do not change
    bare = ops.pack_global(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], N, P, S, innovation=False, **kw)
    assert bare[6] is None and bare[7] is None
    for a, b in ((bare[0], qp), (bare[2], k), (bare[3], vt), (bare[4], pq), (bare[5], pk)):
        assert np.array_equal(_bits(a), _bits(b))


def test_pack_global_rejects_frames_without_patch_tokens():
    from vasc_amd import ops
    x = _bf16((1, 12, 3, 1, 64), 5).cuda()
    with pytest.raises(ValueError, match="patch token"):
        ops.pack_global(x[:, :, 0], x[:, :, 1], x[:, :, 2], 2, 6, 6)


@pytest.mark.parametrize("N,P,S", [(3, 1041, 5), (2, 50, 0), (2, 7, 7)])
def test_restore_bit_exact(N, P, S):
    from vasc_amd import ops
    H, D = 3, 64
    xp = _bf16((2, H, N * (P - S), D), 11)
    xs = _bf16((2, H, N * S, D), 12) if S else None
    out = ops.restore_tokens(xp.cuda(), xs.cuda() if S else None, N, P, S)
    re = xp.float().numpy() if not S else np.concatenate([xp.float().numpy(), xs.float().numpy()], axis=2)
    ref = OL.restore_to_frame_major(re, N, P, S).transpose(0, 2, 1, 3).reshape(2, N * P, H * D)
    assert np.array_equal(_to_np(out), ref)


def test_global_attn_patch_and_special_in_one_launch():
    """Patch rows: bit-identical to the block-sparse entry point on the same
    lists; special rows: bit-identical to the dense entry point and within
    tolerance of the float64 oracle."""
    from vasc_amd import ops
    B, H, Np, Ns, D = 1, 3, 2000, 150, 64
    Tk = Np + Ns
    q = _bf16((B, H, Np, D), 21).cuda()
    qs = _bf16((B, H, Ns, D), 22).cuda()
    k = _bf16((B, H, Tk, D), 23).cuda()
    v = _bf16((B, H, Tk, D), 24).cuda()
    nkb, qb = math.ceil(Tk / 64), math.ceil(Np / 128)
    rng = np.random.default_rng(25)
    idx = np.full((B, H, qb, nkb), -1, np.int32)
    cnt = rng.integers(1, nkb + 1, size=(B, H, qb)).astype(np.int32)
    for bb in range(B):
        for h in range(H):
            for i in range(qb):
                idx[bb, h, i, : cnt[bb, h, i]] = np.sort(rng.choice(nkb, cnt[bb, h, i], replace=False))
    index, count = torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()
    vt = ops.pack_v(v)
    o_p, o_s = ops.global_attn(q, qs, k, vt, index, count)
    assert np.array_equal(_bits(o_p), _bits(ops.block_sparse_attn(q, k, vt, index, count)))
    assert np.array_equal(_bits(o_s), _bits(ops.dense_attn(qs, k, vt)))
    dl, dc = OA.dense_lists(B, H, Ns, Tk)
    ref = OA.block_sparse_attention(qs.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                    dl, dc)
    err = np.abs(_to_np(o_s) - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    o_p2, none = ops.global_attn(q, None, k, vt, index, count)
    assert none is None and np.array_equal(_bits(o_p2), _bits(o_p))


@pytest.mark.parametrize("N,P,S,H,B", [(3, 1041, 5, 2, 1), (4, 70, 0, 1, 1), (2, 7, 7 - 1, 2, 1), (2, 37, 4, 2, 2)])
def test_global_attn_tokens_equals_attention_then_restore(N, P, S, H, B):
    """vasc_global_attn_tokens_fwd writes every result on its frame-major
    token row: bit-identical to vasc_global_attn_fwd followed by the restore
    kernel (frames with and without special tokens, a ragged last block, a
    batch of two)."""
    from vasc_amd import ops
    D = 64
    Np, Ns, Tk = N * (P - S), N * S, N * P
    q = _bf16((B, H, Np, D), 31).cuda()
    qs = _bf16((B, H, Ns, D), 32).cuda() if S else None
    k = _bf16((B, H, Tk, D), 33).cuda()
    v = _bf16((B, H, Tk, D), 34).cuda()
    nkb, qb = math.ceil(Tk / 64), math.ceil(Np / 128)
    rng = np.random.default_rng(35)
    idx = np.full((B, H, qb, nkb), -1, np.int32)
    cnt = rng.integers(1, nkb + 1, size=(B, H, qb)).astype(np.int32)
    for bb in range(B):
        for h in range(H):
            for i in range(qb):
                idx[bb, h, i, : cnt[bb, h, i]] = np.sort(rng.choice(nkb, cnt[bb, h, i], replace=False))
    index, count = torch.from_numpy(idx).cuda(), torch.from_numpy(cnt).cuda()
    vt = ops.pack_v(v)
    o_p, o_s = ops.global_attn(q, qs, k, vt, index, count)
    ref = ops.restore_tokens(o_p, o_s, N, P, S)
    got = ops.global_attn_tokens(q, qs, k, vt, index, count, N, P, S)
    assert got.shape == (B, Tk, H * D)
    assert np.array_equal(_bits(got), _bits(ref))


def test_global_layer_sparse_matches_oracle_layer():
    """The fused layer forward (layout kernel with LayerNorm + rotary, pooled
    predictor, Top-K selection, one attention launch, restore) against the
    oracle's layer on the same module: the index lists come from the GPU
    selection and the oracle recomputes attention over exactly those blocks."""
    import os
    from vasc_amd import ops
    from vasc_amd.aggregator import Attention, RotaryPositionEmbedding2D
    from vasc_amd.attention import adaptive_sparse_attention_forward, predict_attention
    from vasc_amd.sparse_wrapper import get_block_mask

    torch.manual_seed(31)
    N, Hp, Wp, S, heads, dim = 4, 11, 13, 5, 4, 256
    P = Hp * Wp + S
    m = Attention(dim, heads, rope=RotaryPositionEmbedding2D()).cuda().to(torch.bfloat16)
    with torch.no_grad():
        m.q_norm.weight.normal_(1.0, 0.2)
        m.k_norm.bias.normal_(0.0, 0.2)
    x = torch.randn(1, N * P, dim, device="cuda", dtype=torch.bfloat16)
    ys, xs = torch.meshgrid(torch.arange(Hp), torch.arange(Wp), indexing="ij")
    frame_pos = torch.cat([torch.zeros(S, 2, dtype=torch.long), torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1])
    pos = frame_pos.repeat(N, 1).unsqueeze(0).cuda()
    saved = {kk: os.environ.pop(kk) for kk in list(os.environ) if kk.startswith("SPARSE_VGGT_")}
    try:
        os.environ["SPARSE_VGGT_OFFICIAL_MASK"] = "1"
        with torch.no_grad():
            out = adaptive_sparse_attention_forward(m, x, pos, sparse_ratio=0.5, num_special_tokens=S,
                                                    num_heads=heads, routing_state={})
            qkv = m.qkv(x)
            cos, sin = m.rope.tables(dim // heads, "cuda")
            qp, qsp, kre, vre = OL.pack_layer(
                qkv.float().cpu().numpy(), N, P, S, heads,
                q_norm=(m.q_norm.weight.float().cpu().numpy(), m.q_norm.bias.float().cpu().numpy(), m.q_norm.eps),
                k_norm=(m.k_norm.weight.float().cpu().numpy(), m.k_norm.bias.float().cpu().numpy(), m.k_norm.eps),
                pos=pos[0].cpu().numpy(), tables=(cos.cpu().numpy(), sin.cpu().numpy()))
            # the selection the layer made, from the GPU pooled scores of the same packed q/k
            gq, _, gk, _ = ops.pack_qkv(*(qkv.view(1, N * P, 3, heads, dim // heads)[:, :, i] for i in range(3)),
                                        N, P, S, q_norm=(m.q_norm.weight, m.q_norm.bias, m.q_norm.eps),
                                        k_norm=(m.k_norm.weight, m.k_norm.bias, m.k_norm.eps), pos=pos,
                                        rope_tables=(cos, sin))
            n_patch = N * (P - S)
            score = predict_attention(gq, gk[:, :, :n_patch])
            sink = math.ceil(N * P / 64) - score.shape[-1]
            mask = get_block_mask(score, sink, sparse_ratio=0.5)
    finally:
        os.environ.pop("SPARSE_VGGT_OFFICIAL_MASK", None)
        os.environ.update(saved)
    mk = mask.cpu().numpy()
    Qb = mk.shape[2]
    W = mk.shape[3]
    idx = np.full((1, heads, Qb, W), -1, np.int32)
    cnt = mk.sum(-1).astype(np.int32)
    for h in range(heads):
        for i in range(Qb):
            sel = np.nonzero(mk[0, h, i])[0]
            idx[0, h, i, : sel.size] = sel
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).float().numpy()  # noqa: E731  (inputs as the GPU sees them)
    o_p = OA.block_sparse_attention(bf(qp), bf(kre), bf(vre), idx, cnt)
    dl, dc = OA.dense_lists(1, heads, N * S, N * P)
    o_s = OA.block_sparse_attention(bf(qsp), bf(kre), bf(vre), dl, dc)
    o = OL.restore_to_frame_major(np.concatenate([o_p, o_s], axis=2), N, P, S)
    o = torch.from_numpy(o.transpose(0, 2, 1, 3).reshape(1, N * P, dim)).to(torch.bfloat16).cuda()
    with torch.no_grad():
        ref = m.proj(o).float()
    err = (out.float() - ref).abs()
    assert err.max() < 6e-2 and err.mean() < 6e-3, (err.max().item(), err.mean().item())


@pytest.mark.parametrize("backbone", ["vggt", "pi3"])
def test_global_layer_vasc_chain_matches_oracle(backbone, monkeypatch):
    """Three chained global layers through adaptive_sparse_attention_forward in
    the release vasc mode, sharing one routing_state (the cross-layer ledger).
    Each layer's index lists are bit-exact with the oracle's VASC selector
    chain fed the layer's GPU pooled scores and innovations (VGGT: official
    mask; Pi3: the mixed tail block forced and protected), and each layer's
    output matches the oracle layer (norms, rotary, reorder, attention over
    those lists, special queries over every key, restore) through proj."""
    import os
    from oracle import pooling as OP
    from oracle import selector as OS
    from vasc_amd import launcher, sparse_wrapper
    from vasc_amd.aggregator import Attention, RotaryPositionEmbedding2D
    from vasc_amd.attention import adaptive_sparse_attention_forward

    recorded = []
    original = sparse_wrapper._select_for_layer

    def record(key, value, pooled_score, *args, **kwargs):
        sel, total = original(key, value, pooled_score, *args, **kwargs)
        assert value is None, "the fused layout hands over the V tiles, not the values"
        recorded.append({"prob": pooled_score.clone(), "innovation": kwargs["innovation"].clone(),
                         "index": sel["index"].clone(), "count": sel["count"].clone()})
        return sel, total

    monkeypatch.setattr(sparse_wrapper, "_select_for_layer", record)
    torch.manual_seed(41)
    N, Hp, Wp, S, heads, dim = 4, 11, 13, 5, 4, 256
    P = Hp * Wp + S
    n_patch, n_total = N * (P - S), N * P
    assert n_patch % 64 != 0  # a mixed tail block
    ys, xs = torch.meshgrid(torch.arange(Hp), torch.arange(Wp), indexing="ij")
    frame_pos = torch.cat([torch.zeros(S, 2, dtype=torch.long), torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1])
    pos = frame_pos.repeat(N, 1).unsqueeze(0).cuda()
    rope = RotaryPositionEmbedding2D()
    mods, xs_in, outs = [], [], []
    routing_state: dict = {}
    saved = {kk: os.environ.pop(kk) for kk in list(os.environ) if kk.startswith("SPARSE_VGGT_")}
    try:
        os.environ.update(launcher.method_environment(backbone, "vasc"))
        official = backbone == "vggt"
        with torch.no_grad():
            for layer in range(3):
                m = Attention(dim, heads, rope=rope).cuda().to(torch.bfloat16)
                m.q_norm.weight.normal_(1.0, 0.2)
                m.k_norm.bias.normal_(0.0, 0.2)
                x = torch.randn(1, n_total, dim, device="cuda", dtype=torch.bfloat16)
                outs.append(adaptive_sparse_attention_forward(m, x, pos, sparse_ratio=0.5, num_special_tokens=S,
                                                              num_heads=heads, layer_idx=layer,
                                                              routing_state=routing_state))
                mods.append(m)
                xs_in.append(x)
    finally:
        for kk in [kk for kk in os.environ if kk.startswith("SPARSE_VGGT_")]:
            del os.environ[kk]
        os.environ.update(saved)
    assert len(recorded) == 3
    state: dict = {}
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).float().numpy()  # noqa: E731
    for layer, (rec, m, x, out) in enumerate(zip(recorded, mods, xs_in, outs)):
        iota = rec["innovation"].cpu().numpy()
        final, _ = OS.layer_selection(rec["prob"].cpu().numpy(), mode="vasc", sparse_ratio=0.5, patch_tokens=n_patch,
                                      total_tokens=n_total, official_mask=official, state=state, layer_idx=layer,
                                      iota=iota)
        idx, cnt = OS.index_lists(final)
        got_i, got_c = rec["index"].cpu().numpy(), rec["count"].cpu().numpy()
        assert np.array_equal(got_c, cnt), f"layer {layer}: counts differ from the oracle"
        for r, (a, b) in enumerate(zip(got_i.reshape(-1, got_i.shape[-1]), idx.reshape(-1, idx.shape[-1]))):
            n = cnt.reshape(-1)[r]
            assert np.array_equal(a[:n], b[:n]), f"layer {layer}: index list of row {r} differs from the oracle"
        if not official:
            kb = rec["prob"].shape[-1]
            assert (got_i == kb - 1).any(-1).all(), "the protected mixed tail block is in every list"
        with torch.no_grad():
            qkv = m.qkv(x)
            cos, sin = m.rope.tables(dim // heads, "cuda")
            qp, qsp, kre, vre = OL.pack_layer(
                qkv.float().cpu().numpy(), N, P, S, heads,
                q_norm=(m.q_norm.weight.float().cpu().numpy(), m.q_norm.bias.float().cpu().numpy(), m.q_norm.eps),
                k_norm=(m.k_norm.weight.float().cpu().numpy(), m.k_norm.bias.float().cpu().numpy(), m.k_norm.eps),
                pos=pos[0].cpu().numpy(), tables=(cos.cpu().numpy(), sin.cpu().numpy()))
        # the layer's innovation against the oracle's from the oracle's packed
        # values: their bf16 block means may differ by one rounding per
        # element, which moves 0.5 ||l - r|| / sqrt(D) by at most half the
        # norm of those roundings (triangle inequality), plus float32 error
        ref_pv = OP.pool_blocks(bf(vre)[:, :, :n_patch], 64, round_bf16=True)
        ref_iota = OS.innovation(ref_pv)
        sp = OP.bf16_spacing(np.abs(ref_pv) * (1 + 2.0 ** -7))  # the larger gap when a mean rounds up a binade
        if sp.shape[-2] % 2:
            sp = np.concatenate([sp, sp[..., -1:, :]], axis=-2)
        step = 0.5 * np.sqrt(((sp[..., 0::2, :] + sp[..., 1::2, :]) ** 2).mean(-1))
        assert (np.abs(iota - ref_iota) <= step + 1e-6 * ref_iota + 1e-30).all(), f"layer {layer}: innovation"
        o_p = OA.block_sparse_attention(bf(qp), bf(kre), bf(vre), got_i, got_c)
        dl, dc = OA.dense_lists(1, heads, N * S, n_total)
        o_s = OA.block_sparse_attention(bf(qsp), bf(kre), bf(vre), dl, dc)
        o = OL.restore_to_frame_major(np.concatenate([o_p, o_s], axis=2), N, P, S)
        o = torch.from_numpy(o.transpose(0, 2, 1, 3).reshape(1, n_total, dim)).to(torch.bfloat16).cuda()
        with torch.no_grad():
            ref = m.proj(o).float()
        err = (out.float() - ref).abs()
        assert err.max() < 6e-2 and err.mean() < 6e-3, (layer, err.max().item(), err.mean().item())
    assert "cosa_value_risk_pair_debt" in routing_state
    # the ledger's QK-order priority is the last layer's cleaned score
    last = recorded[-1]["prob"]
    prio = routing_state["cosa_value_risk_pair_qk_order_priority"]
    assert torch.equal(prio.view(torch.int32), torch.where(last > 0, last, 0.0).view(torch.int32))


def test_pack_norm_parameters_bf16_and_updated_through_data():
    """bf16 LayerNorm parameters are read as they are (identical to their
    float32 values), and a parameter rewritten through ``.data`` (which
    leaves its version counter alone) is seen by the next call."""
    from vasc_amd import ops
    N, P, S, H, D = 2, 70, 5, 3, 64
    x = _bf16((1, N * P, 3 * H * D), 17, 2.0).cuda().view(1, N * P, 3, H, D)
    g = torch.Generator().manual_seed(18)
    w = torch.nn.Parameter((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda())
    b = torch.nn.Parameter((0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda())

    def run(wt, bt):
        return ops.pack_qkv(x[:, :, 0], x[:, :, 1], x[:, :, 2], N, P, S, q_norm=(wt, bt, 1e-6),
                            k_norm=(wt, None, 1e-6))

    first = run(w, b)
    as_f32 = run(w.float(), b.float())
    for a, c in zip(first, as_f32):
        assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    new_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    w.data.copy_(new_w)
    second = run(w, b)
    fresh = run(new_w.clone(), b.detach().clone())
    for a, c in zip(second, fresh):
        assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    assert not torch.equal(first[0].view(torch.int16), second[0].view(torch.int16))
