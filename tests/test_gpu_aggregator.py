"""VGGT/Pi3-shaped aggregators on the HIP kernels.

* dense forward vs a float32 torch restatement of the same blocks (SDPA,
  LayerNorm, rotary embedding in torch): max-abs <= 3e-2 * max|ref| + 3e-2
  (bf16 weights and activations against float32);
* the sparse install at sparsity 0 keeps every block and matches the dense
  forward (same tolerance);
* VASC mode: the ledger is cleared at the start of a forward and settled
  after the last layer, so two forwards on the same input are bit-identical
  and the pending arrival is gone afterwards (finalize, sparse_wrapper.py:
  4101-4177); the per-layer sparsity is recorded when aux_output is on.
"""
import os

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


def _ref_attention(attn, x, pos):
    B, T, C = x.shape
    H = attn.num_heads
    D = C // H
    qkv = F.linear(x, attn.qkv.weight.float(), attn.qkv.bias.float()).view(B, T, 3, H, D).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    q = F.layer_norm(q, (D,), attn.q_norm.weight.float(), attn.q_norm.bias.float(), attn.q_norm.eps)
    k = F.layer_norm(k, (D,), attn.k_norm.weight.float(), attn.k_norm.bias.float(), attn.k_norm.eps)
    q, k = attn.rope(q, pos), attn.rope(k, pos)
    o = F.scaled_dot_product_attention(q, k, v)
    return F.linear(o.transpose(1, 2).reshape(B, T, C), attn.proj.weight.float(), attn.proj.bias.float())


def _ref_block(blk, x, pos):
    ln = lambda m, t: F.layer_norm(t, m.normalized_shape, m.weight.float(), m.bias.float(), m.eps)  # noqa: E731
    x = x + blk.ls1.gamma.float() * _ref_attention(blk.attn, ln(blk.norm1, x), pos)
    h = F.gelu(F.linear(ln(blk.norm2, x), blk.mlp.fc1.weight.float(), blk.mlp.fc1.bias.float()))
    return x + blk.ls2.gamma.float() * F.linear(h, blk.mlp.fc2.weight.float(), blk.mlp.fc2.bias.float())


def _ref_aggregator(agg, images):
    from vasc_amd.aggregator import grid_positions
    B, N, _, Hi, Wi = images.shape
    x = ((images - agg._resnet_mean) / agg._resnet_std).view(B * N, 3, Hi, Wi).float()
    tok = F.conv2d(x, agg.patch_embed.weight.float(), agg.patch_embed.bias.float(), stride=agg.patch_size)
    tok = tok.flatten(2).transpose(1, 2)
    special = [agg._expand(agg.camera_token, B, N), agg._expand(agg.register_token, B, N)]
    tok = torch.cat([*(s.float() for s in special), tok], dim=1)
    P, C = tok.shape[1:]
    pos = grid_positions(B * N, Hi // agg.patch_size, Wi // agg.patch_size, agg.patch_start_idx, images.device)
    for i in range(agg.aa_block_num):
        tok = _ref_block(agg.frame_blocks[i], tok.view(B * N, P, C), pos)
        tok = _ref_block(agg.global_blocks[i], tok.view(B, N * P, C), pos.reshape(B, N * P, 2))
    return tok.view(B, N, P, C)


def _close(out, ref):
    err = (out.float() - ref).abs().max().item()
    assert err <= 3e-2 * ref.abs().max().item() + 3e-2, (err, ref.abs().max().item())


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


def test_dense_aggregator_matches_torch_float32():
    agg = _model(Aggregator, dim=128, depth=2, num_heads=2, mlp_ratio=2.0, intermediate_layer_idx=(1,))
    images = _images()
    with torch.no_grad():
        ref = _ref_aggregator(agg, images)
        outs, start = agg.to(torch.bfloat16)(images)
    assert start == 5 and outs[0] is None and outs[1] is not None
    _close(outs[-1][..., 128:], ref)


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
