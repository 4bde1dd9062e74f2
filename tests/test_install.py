"""Installers of the sparse global attention (CPU: module wiring only)."""
import pytest

from vasc_amd import install
from vasc_amd.aggregator import Aggregator, Pi3Decoder


def _small_vggt():
    return Aggregator(dim=128, depth=3, num_heads=2, mlp_ratio=2.0)


def test_vggt_uniform_install_patches_every_global_block():
    agg, store = install.sparse_aggregator_from_vggt(_small_vggt(), sparse_ratio=0.75, verbose=False)
    state = agg._sparse_routing_state
    assert state == {} and store == {0: None, 1: None, 2: None}
    for i, blk in enumerate(agg.global_blocks):
        fwd = blk.attn.forward
        assert fwd.__self__ is blk.attn and blk.attn._sparse_routing_state is state
        assert fwd.__func__.keywords["layer_idx"] == i and fwd.__func__.keywords["sparse_ratio"] == 0.75
    for blk in agg.frame_blocks:
        assert not hasattr(blk.attn, "_sparse_routing_state")


def test_vggt_layerwise_ratios_and_aux_store():
    agg, store = install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.7, 0.8, 0.9],
                                                               aux_output=True, verbose=False)
    assert store == {0: {}, 1: {}, 2: {}}
    assert [b.attn.forward.__func__.keywords["sparse_ratio"] for b in agg.global_blocks] == [0.7, 0.8, 0.9]
    assert agg.global_blocks[1].attn.forward.__func__.keywords["aux_output_store"] is store[1]
    with pytest.raises(ValueError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.5, 0.5], verbose=False)
    with pytest.raises(ValueError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.5, 1.5, 0.5],
                                                      verbose=False)


def test_research_options_are_refused():
    with pytest.raises(NotImplementedError):
        install.sparse_aggregator_from_vggt(_small_vggt(), sparse_ratio=0.75, use_hilbert=True, verbose=False)
    with pytest.raises(NotImplementedError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), sparse_ratio=0.75, use_radial_layerwise=True,
                                                      verbose=False)
    with pytest.raises(AssertionError):  # neither ratio nor cdf (check_sparse_mode)
        install.sparse_aggregator_from_vggt(_small_vggt(), verbose=False)


def test_pi3_odd_layers_are_global_with_logical_index():
    model = Pi3Decoder(dim=128, depth=6, num_heads=2, mlp_ratio=2.0)
    # the reference checks the uniform mode first (pi3.py:164), so the caller passes sparse_ratio too
    model, store = install.sparse_model_from_pi3(model, sparse_ratio=0.7, layer_sparsity_ratios=[0.6, 0.7, 0.8],
                                                 verbose=False)
    assert sorted(store) == [0, 1, 2]
    for i, blk in enumerate(model.decoder):
        if i % 2:
            kw = blk.attn.forward.__func__.keywords
            assert kw["layer_idx"] == i // 2 and kw["sparse_ratio"] == [0.6, 0.7, 0.8][i // 2]
        else:
            assert not hasattr(blk.attn, "_sparse_routing_state")
    with pytest.raises(ValueError):
        install.sparse_model_from_pi3(Pi3Decoder(dim=128, depth=6, num_heads=2), sparse_ratio=0.5,
                                      layer_sparsity_ratios=[0.5] * 2, verbose=False)


def test_patch_tokens_equal_the_convolution():
    """The runners' patch embedding as one GEMM over non-overlapping patches
    equals the strided convolution (ragged borders dropped as the conv does);
    other convolutions fall back to the module itself."""
    import torch

    from vasc_amd.aggregator import patch_tokens
    torch.manual_seed(0)
    x = torch.randn(3, 3, 70, 85)
    conv = torch.nn.Conv2d(3, 32, 14, 14)
    ref = conv(x).flatten(2).transpose(1, 2)
    got = patch_tokens(conv, x)
    assert got.shape == ref.shape == (3, 30, 32)
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)
    overlap = torch.nn.Conv2d(3, 8, 4, 2)
    assert torch.equal(patch_tokens(overlap, x), overlap(x).flatten(2).transpose(1, 2))
