"""VGGT/Pi3-shaped aggregators on the HIP kernels.

* dense forward vs a float32 torch restatement of the same blocks (SDPA,
  LayerNorm, rotary embedding in torch), element by element:
  |out - ref| <= 3e-2 * |ref| + 3e-2 * rms(ref) (bf16 activations against
  float32 on the same bf16 weights);
* the sparse install at sparsity 0 keeps every block and matches the dense
  forward (same tolerance);
* VASC mode: the ledger is cleared at the start of a forward and settled
  after the last layer, so two forwards on the same input are bit-identical
  and the pending arrival is gone afterwards (finalize, sparse_wrapper.py:
  4101-4177); the per-layer sparsity is recorded when aux_output is on;
* sparse forwards (VGGT vasc, Pi3 vasc and topk) vs the same float32
  restatement with each global layer restricted to the index lists the GPU
  selection produced (teacher-forced; recorded at the selection call), and
  the recorded lists bit-exact with the oracle selector chain fed the GPU's
  pooled scores and innovations.
"""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from vasc_amd import install, launcher
from vasc_amd.aggregator import Aggregator, Pi3Decoder

pytestmark = pytest.mark.gpu


def _model(cls, **kw):
    torch.manual_seed(0)
    m = cls(**kw)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("gamma"):
                p.fill_(1.0)  # full-strength residual branches: attention errors stay visible
            elif "norm" in name and name.endswith("weight"):
                p.normal_(1.0, 0.1)
    return m.cuda()


def _patch_first(N, P, S, device):
    """Frame-major token index of each position of the [all patches; all
    specials] order the sparse layer uses."""
    f = torch.arange(N, device=device).view(N, 1)
    patch = (f * P + S + torch.arange(P - S, device=device).view(1, -1)).reshape(-1)
    special = (f * P + torch.arange(S, device=device).view(1, -1)).reshape(-1)
    return torch.cat([patch, special])


def _list_mask(index, count, n_patch, n_total):
    """Token mask [B,H,n_patch,n_total] of 128-query x 64-key block lists (patch-first order)."""
    B, H, Qb, W = index.shape
    kbt = -(-n_total // 64)
    live = torch.arange(W, device=index.device).view(1, 1, 1, W) < count.unsqueeze(-1)
    bm = torch.zeros(B, H, Qb, kbt + 1, dtype=torch.bool, device=index.device)
    bm.scatter_(3, torch.where(live, index.long(), kbt), True)
    return bm[..., :kbt].repeat_interleave(128, 2)[:, :, :n_patch].repeat_interleave(64, 3)[..., :n_total]


def _chunked_attention(q, k, v, rows: int = 2048):
    """float32 softmax attention over query chunks (a full score matrix of a
    33 312-token layer would take 71 GB)."""
    kt = k.transpose(-1, -2).contiguous()
    out = torch.empty_like(q)
    scale = q.shape[-1] ** -0.5
    for i in range(0, q.shape[2], rows):
        s = torch.matmul(q[:, :, i:i + rows].contiguous(), kt) * scale
        out[:, :, i:i + rows] = torch.matmul(s.softmax(-1), v)
    return out


def _ref_attention(attn, x, pos, sparse=None):
    """float32 attention of one block; ``sparse = (N, P, S, index, count)``
    restricts the patch queries of a global layer to their listed blocks
    (special-token queries attend to every key)."""
    B, T, C = x.shape
    H = attn.num_heads
    D = C // H
    qkv = F.linear(x, attn.qkv.weight.float(), attn.qkv.bias.float()).view(B, T, 3, H, D).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    q = F.layer_norm(q, (D,), attn.q_norm.weight.float(), attn.q_norm.bias.float(), attn.q_norm.eps)
    k = F.layer_norm(k, (D,), attn.k_norm.weight.float(), attn.k_norm.bias.float(), attn.k_norm.eps)
    q, k = attn.rope(q, pos), attn.rope(k, pos)
    if sparse is None and T > 8192:
        o = _chunked_attention(q, k, v)
    elif sparse is None:
        o = F.scaled_dot_product_attention(q, k, v)
    else:
        N, P, S, index, count = sparse
        n_patch = N * (P - S)
        perm = _patch_first(N, P, S, x.device)
        mask = torch.ones(B, H, T, T, dtype=torch.bool, device=x.device)
        mask[:, :, :n_patch] = _list_mask(index, count, n_patch, T)
        o_re = F.scaled_dot_product_attention(q[:, :, perm], k[:, :, perm], v[:, :, perm], attn_mask=mask)
        o = torch.empty_like(o_re)
        o[:, :, perm] = o_re
    return F.linear(o.transpose(1, 2).reshape(B, T, C), attn.proj.weight.float(), attn.proj.bias.float())


def _ref_block(blk, x, pos, sparse=None):
    ln = lambda m, t: F.layer_norm(t, m.normalized_shape, m.weight.float(), m.bias.float(), m.eps)  # noqa: E731
    x = x + blk.ls1.gamma.float() * _ref_attention(blk.attn, ln(blk.norm1, x), pos, sparse)
    h = F.gelu(F.linear(ln(blk.norm2, x), blk.mlp.fc1.weight.float(), blk.mlp.fc1.bias.float()))
    return x + blk.ls2.gamma.float() * F.linear(h, blk.mlp.fc2.weight.float(), blk.mlp.fc2.bias.float())


def _ref_aggregator(agg, images, lists=None):
    from vasc_amd.aggregator import grid_positions
    B, N, _, Hi, Wi = images.shape
    x = ((images - agg._resnet_mean) / agg._resnet_std).view(B * N, 3, Hi, Wi).float()
    tok = F.conv2d(x, agg.patch_embed.weight.float(), agg.patch_embed.bias.float(), stride=agg.patch_size)
    tok = tok.flatten(2).transpose(1, 2)
    special = [agg._expand(agg.camera_token, B, N), agg._expand(agg.register_token, B, N)]
    tok = torch.cat([*(s.float() for s in special), tok], dim=1)
    P, C = tok.shape[1:]
    pos = grid_positions(B * N, Hi // agg.patch_size, Wi // agg.patch_size, agg.patch_start_idx, images.device)
    S = agg.patch_start_idx
    for i in range(agg.aa_block_num):
        tok = _ref_block(agg.frame_blocks[i], tok.view(B * N, P, C), pos)
        sparse = None if lists is None else (N, P, S, lists[i]["index"], lists[i]["count"])
        tok = _ref_block(agg.global_blocks[i], tok.view(B, N * P, C), pos.reshape(B, N * P, 2), sparse)
    return tok.view(B, N, P, C)


def _ref_pi3(model, images, lists=None):
    """float32 restatement of Pi3Decoder.forward (odd blocks global)."""
    from vasc_amd.aggregator import grid_positions
    B, N, _, Hi, Wi = images.shape
    x = images.view(B * N, 3, Hi, Wi).float()
    hid = F.conv2d(x, model.patch_embed.weight.float(), model.patch_embed.bias.float(), stride=model.patch_size)
    hid = hid.flatten(2).transpose(1, 2)
    reg = model.register_token.float().repeat(B, N, 1, 1).reshape(B * N, *model.register_token.shape[-2:])
    hid = torch.cat([reg, hid], dim=1)
    P, C = hid.shape[1:]
    S = model.patch_start_idx
    pos = grid_positions(B * N, Hi // model.patch_size, Wi // model.patch_size, S, images.device)
    final, g = [], 0
    for i, blk in enumerate(model.decoder):
        if i % 2 == 0:
            hid = _ref_block(blk, hid.reshape(B * N, P, C), pos)
        else:
            sparse = None if lists is None else (N, P, S, lists[g]["index"], lists[g]["count"])
            hid = _ref_block(blk, hid.reshape(B, N * P, C), pos.reshape(B, N * P, 2), sparse)
            g += 1
        if i + 1 in (len(model.decoder) - 1, len(model.decoder)):
            final.append(hid.reshape(B * N, P, C))
    return torch.cat(final, dim=-1)


class _Recorder:
    """Records, per sparse global layer, the pooled scores, the values' pair
    innovation the selection was given (or the value tensor, when the
    caller handed the values instead) and the index lists it produced."""

    def __init__(self, monkeypatch):
        from vasc_amd import sparse_wrapper
        self.layers = []
        original = sparse_wrapper._select_for_layer

        def record(key, value, pooled_score, *args, **kwargs):
            sel, total = original(key, value, pooled_score, *args, **kwargs)
            inn = kwargs.get("innovation")
            self.layers.append({"prob": pooled_score.clone(), "value": None if value is None else value.clone(),
                                "innovation": None if inn is None else inn.clone(),
                                "index": sel["index"].clone(), "count": sel["count"].clone()})
            return sel, total

        monkeypatch.setattr(sparse_wrapper, "_select_for_layer", record)


def _oracle_chain(layers, n_patch, n_total, ratios, mode, official):
    """The recorded lists vs the oracle selection chain on the recorded scores."""
    from oracle import selector as OS
    from vasc_amd import ops
    state: dict = {}
    for li, rec in enumerate(layers):
        iota = None
        if mode == "vasc":
            inn = rec["innovation"]
            if inn is None:
                inn = ops.pool_qkv(v=rec["value"][..., :n_patch, :])[3]
            iota = inn.cpu().numpy()
        final, _ = OS.layer_selection(rec["prob"].cpu().numpy(), mode=mode, sparse_ratio=ratios[li],
                                      patch_tokens=n_patch, total_tokens=n_total, official_mask=official,
                                      state=state, layer_idx=li, iota=iota)
        idx, cnt = OS.index_lists(final)
        got_i, got_c = rec["index"].cpu().numpy(), rec["count"].cpu().numpy()
        assert np.array_equal(got_c, cnt), f"layer {li}: counts differ from the oracle"
        for r in range(cnt.size):
            n = cnt.reshape(-1)[r]
            a = got_i.reshape(-1, got_i.shape[-1])[r, :n]
            assert np.array_equal(a, idx.reshape(-1, idx.shape[-1])[r, :n]), f"layer {li}: row {r}"


def _close(out, ref, rtol: float = 3e-2, atol: float = 3e-2):
    """Element-wise |out - ref| <= rtol*|ref| + atol*rms(ref): a few bf16
    roundings (2^-8 relative each) per block, on every element, with the
    row-independent floor for elements near zero."""
    out, ref = out.float(), ref.float()
    rms = ref.square().mean().sqrt().item()
    err = (out - ref).abs()
    worst = (err / (rtol * ref.abs() + atol * rms)).max().item()
    print(f"max-abs {err.max().item():.3e}, mean-abs {err.mean().item():.3e}, rms(ref) {rms:.3e}, "
          f"worst error / bound {worst:.3f}")
    assert worst <= 1.0, worst


def _images(N=3, H=70, W=84, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(1, N, 3, H, W, generator=g).cuda()


class _Env:
    def __init__(self, backbone, mode):
        self.env = launcher.method_environment(backbone, mode)

    def __enter__(self):
        self.saved = {k: os.environ.pop(k) for k in list(os.environ) if k.startswith("SPARSE_VGGT_")}
        os.environ.update(self.env)

    def __exit__(self, *exc):
        for k in list(os.environ):
            if k.startswith("SPARSE_VGGT_"):
                del os.environ[k]
        os.environ.update(self.saved)


@pytest.mark.parametrize("dim", [128, 512])
def test_dense_aggregator_matches_torch_float32(dim):
    """dim 512 runs the fused residual + LayerNorm passes (vasc_residual_norm)
    between the sub-layers; dim 128 the separate torch ops."""
    agg = _model(Aggregator, dim=dim, depth=2, num_heads=dim // 64, mlp_ratio=2.0, intermediate_layer_idx=(1,))
    images = _images()
    with torch.no_grad():
        ref = _ref_aggregator(agg, images)
        outs, start = agg.to(torch.bfloat16)(images)
    assert start == 5 and outs[0] is None and outs[1] is not None
    _close(outs[-1][..., dim:], ref)


def test_sparse_install_at_zero_sparsity_is_dense():
    agg = _model(Aggregator, dim=128, depth=2, num_heads=2, mlp_ratio=2.0, intermediate_layer_idx=(1,))
    agg = agg.to(torch.bfloat16)
    images = _images(N=4)
    with torch.no_grad():
        dense, _ = agg(images)
        with _Env("vggt", "topk"):
            install.sparse_aggregator_from_vggt(agg, sparse_ratio=0.0, verbose=False)
            sparse, _ = agg(images)
    _close(sparse[-1], dense[-1].float())


def test_vasc_forward_clears_and_settles_the_ledger():
    agg = _model(Aggregator, dim=128, depth=3, num_heads=2, mlp_ratio=2.0, intermediate_layer_idx=(2,))
    agg = agg.to(torch.bfloat16)
    images = _images(N=6, H=112, W=126)
    with torch.no_grad(), _Env("vggt", "vasc"):
        _, store = install.sparse_aggregator_from_vggt(agg, sparse_ratio=0.75, aux_output=True, verbose=False)
        a, _ = agg(images)
        state = dict(agg._sparse_routing_state)
        b, _ = agg(images)
    assert torch.equal(a[-1], b[-1])
    assert "cosa_value_risk_pair_debt" in state and "cosa_value_risk_pair_pending_arrival" not in state
    for i in range(3):
        s = float(store[i]["sparsity"])
        assert 0.0 < s < 1.0, s


def test_pi3_decoder_topk_runs_and_zero_sparsity_is_dense():
    model = _model(Pi3Decoder, dim=128, depth=4, num_heads=2, mlp_ratio=2.0).to(torch.bfloat16)
    images = _images(N=3)
    with torch.no_grad():
        dense, pos = model(images)
        with _Env("pi3", "topk"):
            install.sparse_model_from_pi3(model, sparse_ratio=0.0, verbose=False)
            sparse, _ = model(images)
    assert pos.shape == (3, 35, 2)
    _close(sparse, dense.float())


@pytest.mark.parametrize("dim", [128, 512])
def test_vasc_aggregator_matches_torch_float32_on_its_lists(dim, monkeypatch):
    """VGGT-shaped aggregator in vasc mode with the structural-style per-layer
    ratios: output vs the float32 restatement over the recorded lists, and the
    lists vs the oracle's VASC chain (official mask: no forced tail)."""
    agg = _model(Aggregator, dim=dim, depth=3, num_heads=dim // 64, mlp_ratio=2.0, intermediate_layer_idx=(2,))
    images = _images(N=6, H=112, W=126)
    ratios = [0.75, 0.6, 0.8]
    rec = _Recorder(monkeypatch)
    with torch.no_grad():
        agg = agg.to(torch.bfloat16)
        with _Env("vggt", "vasc"):
            install.sparse_aggregator_from_vggt_layerwise(agg, layer_sparsity_ratios=ratios, verbose=False)
            outs, _ = agg(images)
        assert len(rec.layers) == 3
        P = 5 + 8 * 9
        _oracle_chain(rec.layers, 6 * (P - 5), 6 * P, ratios, "vasc", official=True)
        for r in rec.layers:  # the lists are sparse: some blocks left out in every layer
            assert int(r["count"].sum()) < r["count"].numel() * (-(-6 * P // 64))
        ref = _ref_aggregator(agg, images, rec.layers)
    _close(outs[-1][..., dim:], ref)


@pytest.mark.parametrize("mode,dim", [("vasc", 128), ("topk", 128), ("vasc", 512)])
def test_pi3_decoder_sparse_matches_torch_float32_on_its_lists(mode, dim, monkeypatch):
    """Pi3-shaped decoder (6 blocks, odd ones global, 5 register tokens, the
    mixed tail protected): output vs the float32 restatement over the recorded
    lists, lists vs the oracle chain; dense vs the restatement without lists."""
    model = _model(Pi3Decoder, dim=dim, depth=6, num_heads=dim // 64, mlp_ratio=2.0).to(torch.bfloat16)
    images = _images(N=5, H=98, W=126, seed=3)
    P = 5 + 7 * 9
    rec = _Recorder(monkeypatch)
    with torch.no_grad():
        dense, _ = model(images)
        _close(dense, _ref_pi3(model, images))
        with _Env("pi3", mode):
            install.sparse_model_from_pi3(model, sparse_ratio=0.75, verbose=False)
            sparse, _ = model(images)
        assert len(rec.layers) == 3
        _oracle_chain(rec.layers, 5 * (P - 5), 5 * P, [0.75] * 3, mode, official=False)
        ref = _ref_pi3(model, images, rec.layers)
    _close(sparse, ref)



def test_c2_width_and_length_blocks():
    """Four frame and four global blocks at config 2's width and sequence
    length (dim 1024, 16 heads, MLP 4096, 32 frames at 392x518: 33 312 global
    tokens): the dense bf16 forward against the float32 restatement; the
    sparse install at sparsity 0 against the dense forward; the vasc forward
    at the structural profile's first four ratios finite and bit-identical
    over two forwards (the ledger is cleared per forward)."""
    images = _images(N=32, H=392, W=518, seed=2)
    agg = _model(Aggregator, dim=1024, depth=4, num_heads=16, mlp_ratio=4.0, intermediate_layer_idx=(3,))
    agg = agg.to(torch.bfloat16)
    with torch.no_grad():
        dense, _ = agg(images)
        ref = _ref_aggregator(agg, images)
        # 16 residual updates of a 1024-wide stream (the small cases above run 4 to 12)
        _close(dense[-1][..., 1024:], ref, rtol=5e-2, atol=5e-2)
        del ref
        with _Env("vggt", "topk"):
            install.sparse_aggregator_from_vggt(agg, sparse_ratio=0.0, verbose=False)
            zero, _ = agg(images)
        # the sparse kernel over full lists sums keys in [patch; special] order, the dense one in
        # frame order: bf16 roundings apart, as the float32 comparison above
        _close(zero[-1], dense[-1], rtol=5e-2, atol=5e-2)
    del agg, zero
    agg = _model(Aggregator, dim=1024, depth=4, num_heads=16, mlp_ratio=4.0, intermediate_layer_idx=(3,))
    agg = agg.to(torch.bfloat16)
    ratios = launcher.layer_sparsity("vggt", 0.75, "paper")[:4]
    with torch.no_grad(), _Env("vggt", "vasc"):
        _, store = install.sparse_aggregator_from_vggt_layerwise(agg, layer_sparsity_ratios=ratios, aux_output=True,
                                                                verbose=False)
        a, _ = agg(images)
        b, _ = agg(images)
    assert torch.isfinite(a[-1]).all()
    assert torch.equal(a[-1], b[-1])
    for i in range(4):  # 120 of 518 patch blocks plus 3 sink blocks per row
        assert abs(float(store[i]["sparsity"]) - (1 - 123 / 521)) < 1e-6, store[i]["sparsity"]
    d = (a[-1].float() - dense[-1].float()).abs()
    print(f"vasc vs dense after 4 global blocks: max-abs {d.max().item():.3e} mean-abs {d.mean().item():.3e}")
